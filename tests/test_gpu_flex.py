"""The FlexAttention-style front end on the GPU: flex_attention with the
reference's own FlexAttention descriptions (extra_bench.py:85-95) against the
callables evaluated literally (oracle/flex.py), the compiled call against
attention() with the fitted parameters (bit-identical: the same kernel), the
sigmoid / ReLU normalisers, grouped-query K/V, lse and gradients."""
import pytest
import torch

from chia_proj_amd import attention, gate
from chia_proj_amd.flex import create_block_mask, fit_score_mod, flex_attention, flex_params
from flex_cases import FLEX_REF, H_REF, SLOPES, TEMPS, causal
from oracle.flex import flex_ref

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(msg):
    print(msg, flush=True)


def _qkv(B, H, Hkv, S, D, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    q = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16)
    k, v = (torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16) for _ in range(2))
    return q, k, v


def _gate(ref, got, scale_aware=False):
    for b in range(ref.shape[0]):
        for h in range(ref.shape[1]):
            res = gate.north_star_gate(ref[b, h], got[b, h].float().cpu(), scale_aware=scale_aware)
            assert res.ok, (b, h, res.status, res.stats)


@pytest.mark.parametrize("op,score_mod,mask_mod", FLEX_REF, ids=[r[0] for r in FLEX_REF])
def test_reference_flex_descriptions(op, score_mod, mask_mod):
    _say(f"[flex] {op}")
    S = 1100
    q, k, v = _qkv(1, H_REF, H_REF, S, 64, 17)
    bm = create_block_mask(mask_mod, 1, H_REF, S, S, device=DEV)
    qd, kd, vd = (t.to(DEV) for t in (q, k, v))
    o = flex_attention(qd, kd, vd, score_mod=score_mod, block_mask=bm)
    params, _ = flex_params(tuple(q.shape), score_mod, bm)
    assert torch.equal(o, attention(qd, kd, vd, **params))
    _gate(flex_ref(q, k, v, score_mod, mask_mod), o)


@pytest.mark.parametrize("norm,kw", [("sigmoid", dict(bias=-2.0)), ("relu", dict(post_scale=0.01))])
def test_sigmoid_and_relu(norm, kw):
    _say(f"[flex] {norm}")
    S, H = 700, 4
    q, k, v = _qkv(2, H, H, S, 64, 23)
    temps = torch.tensor([0.5, 1.0, 1.5, 2.0])
    mod = lambda s, b, h, qi, kj: torch.tanh((s * temps[h]) / 20.0) * 20.0  # noqa: E731
    mask = lambda b, h, qi, kj: (kj <= qi) & (qi - kj < 300)  # noqa: E731
    bm = create_block_mask(mask, None, None, S, S)
    o = flex_attention(*(t.to(DEV) for t in (q, k, v)), score_mod=mod, block_mask=bm, norm=norm, **kw)
    # unnormalised sigmoid output grows like sqrt(visible keys): the scale-aware gate
    _gate(flex_ref(q, k, v, mod, mask, norm=norm, **kw), o, scale_aware=norm == "sigmoid")


def test_grouped_query_and_lse():
    _say("[flex] gqa + lse")
    S, H, Hkv = 520, 8, 2
    q, k, v = _qkv(1, H, Hkv, S, 128, 29)
    slopes = torch.linspace(0.01, 0.2, H)
    mod = lambda s, b, h, qi, kj: s + slopes[h] * (kj - qi) + 0.75  # noqa: E731  (offset: o unchanged, lse shifted)
    fitted = fit_score_mod(mod, H, S)
    bm = create_block_mask(causal, None, None, S, S)
    o, lse = flex_attention(*(t.to(DEV) for t in (q, k, v)), score_mod=fitted, block_mask=bm, enable_gqa=True,
                            return_lse=True)
    _gate(flex_ref(q, k, v, mod, causal), o)
    # lse_i = log sum_j exp(s'_ij) over visible keys, float64 restatement
    rep = H // Hkv
    qf, kf = q.double(), k.double().repeat_interleave(rep, 1)
    s = (qf @ kf.transpose(-2, -1)) / 128 ** 0.5
    i, j = torch.arange(S).view(-1, 1), torch.arange(S).view(1, -1)
    s = s + slopes.double().view(1, H, 1, 1) * (j - i) + 0.75
    ref = torch.logsumexp(s.masked_fill(j > i, float("-inf")), -1)
    # the kernel's row sum adds the bf16-rounded weights that also multiply V
    # (|relative rounding| <= 2^-9 each), so lse may differ by up to ln(1 + 2^-9);
    # the bound below allows twice that
    assert (lse.double().cpu() - ref).abs().max().item() < 2 * 1.953e-3


def test_gradients_through_flex_attention():
    _say("[flex] grad")
    S, H = 300, 4
    q, k, v = _qkv(1, H, H, S, 64, 31)
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(32)).to(torch.bfloat16)
    temps = torch.tensor([0.6, 0.9, 1.2, 1.5])
    mod = lambda s, b, h, qi, kj: s * temps[h]  # noqa: E731
    mask = lambda b, h, qi, kj: (qi // 64 == kj // 64)  # noqa: E731
    bm = create_block_mask(mask, None, None, S, S)
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    flex_attention(qg, kg, vg, score_mod=mod, block_mask=bm).backward(do.to(DEV))
    qf, kf, vf = (t.float().requires_grad_(True) for t in (q, k, v))
    flex_ref(qf, kf, vf, mod, mask).backward(do.float())
    for g, r in ((qg.grad, qf.grad), (kg.grad, kf.grad), (vg.grad, vf.grad)):
        err = (g.float().cpu() - r).abs()
        m = r.abs().max().item()
        assert err.max().item() <= 1e-2 * m and err.mean().item() <= 1e-3 * m
