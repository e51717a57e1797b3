"""CPU pins of oracle/fp8.py: torch's e4m3 cast is the OCP e4m3fn format the
gfx950 FP8 matrix path reads (bias 7, 3 mantissa bits, max 448, round to
nearest even), the emulation without its weight rounding is the generic
oracle, and quantize_fp8 round-trips within half an e4m3 step."""
import pytest
import torch

from chia_proj_amd import quantize_fp8
from oracle.fp8 import e4m3_round, fp8_emulated, fp8_ref


def test_e4m3_format():
    bits = lambda x: int(torch.tensor([x]).to(torch.float8_e4m3fn).view(torch.uint8))  # noqa: E731
    assert bits(1.0) == 0x38 and bits(-2.0) == 0xC0 and bits(448.0) == 0x7E
    assert bits(2.0 ** -6) == 0x08 and bits(2.0 ** -9) == 0x01           # smallest normal, smallest subnormal
    assert e4m3_round(torch.tensor([1.0625])).item() == 1.0              # tie to even (1.0 | 1.125)
    assert e4m3_round(torch.tensor([1.1875])).item() == 1.25             # tie to even (1.125 | 1.25)
    assert e4m3_round(torch.tensor([300.0])).item() == 288.0             # step 32 above 256


def _q8(seed, shape=(1, 2, 96, 64)):
    g = torch.Generator().manual_seed(seed)
    return [quantize_fp8(torch.randn(shape, generator=g)) for _ in range(3)]


@pytest.mark.parametrize("kw", [dict(causal=True), dict(norm="sigmoid", causal=False, bias=-2.0),
                                dict(norm="relu", causal=True, window=20, post_scale=0.1),
                                dict(causal=True, alibi_slopes=[0.1, 0.3], softcap=5.0, dilation=2)])
def test_emulation_error_is_the_weight_rounding(kw, monkeypatch):
    (q8, qd), (k8, kd), (v8, vd) = _q8(1)
    ref = fp8_ref(q8, k8, v8, qd, kd, vd, **kw)
    emu = fp8_emulated(q8, k8, v8, qd, kd, vd, **kw)
    err = (emu - ref).abs() / max(1.0, ref.abs().max().item())
    # e4m3 has 3 mantissa bits: a weight moves by at most 2^-4 of itself, so o by at
    # most 2^-4 of sum |w v|; on random data far less
    assert err.max().item() < 2 ** -4 and err.mean().item() < 0.01
    # without the weight rounding the emulation is the exact computation (up to bf16 output rounding)
    import oracle.fp8 as f
    monkeypatch.setattr(f, "e4m3_round", lambda x: x)
    exact = f.fp8_emulated(q8, k8, v8, qd, kd, vd, **kw)
    assert (exact - ref).abs().max().item() <= 1e-2 * max(1.0, ref.abs().max().item())


def test_quantize_round_trip():
    x = torch.randn(1000, generator=torch.Generator().manual_seed(3)) * 7
    x8, d = quantize_fp8(x)
    assert x8.dtype == torch.float8_e4m3fn and abs(d - x.abs().max().item() / 448.0) < 1e-12
    back = x8.float() * d
    assert ((back - x).abs() <= (x.abs() * 2 ** -4) + 2 ** -9 * d).all()


def test_e5m2_format_and_round_trip():
    """torch.float8_e5m2 is OCP e5m2 (bias 15, 2 mantissa bits, max 57344): the
    storage format 1 of chia_attn_fwd_fp8; quantize_fp8 maps max |x| to 57344."""
    bits = lambda x: int(torch.tensor([x]).to(torch.float8_e5m2).view(torch.uint8))  # noqa: E731
    assert bits(1.0) == 0x3C and bits(-2.0) == 0xC0 and bits(57344.0) == 0x7B
    assert bits(2.0 ** -14) == 0x04 and bits(2.0 ** -16) == 0x01          # smallest normal, smallest subnormal
    x = torch.randn(1000, generator=torch.Generator().manual_seed(4)) * 3
    x8, d = quantize_fp8(x, dtype=torch.float8_e5m2)
    assert x8.dtype == torch.float8_e5m2 and abs(d - x.abs().max().item() / 57344.0) < 1e-12
    back = x8.float() * d
    assert ((back - x).abs() <= (x.abs() * 2 ** -3) + 2 ** -17 * d).all()
    with pytest.raises(TypeError):
        quantize_fp8(x, dtype=torch.float16)


def test_mixed_formats_are_rejected_before_any_launch():
    from chia_proj_amd import attention_fp8
    q = torch.zeros(1, 1, 4, 64).to(torch.float8_e4m3fn)
    k = torch.zeros(1, 1, 4, 64).to(torch.float8_e5m2)
    with pytest.raises(TypeError):
        attention_fp8(q, k, k)
    with pytest.raises(TypeError):
        attention_fp8(q.float(), q, q)


def test_quantize_empty_tensor():
    x8, d = quantize_fp8(torch.empty(0, 2, 64))
    assert x8.shape == (0, 2, 64) and d == 1.0
