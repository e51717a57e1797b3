"""Pins for the CPU oracle (oracle/): every check below is independent of the
oracle's own formulas, so a dropped term, wrong sign, wrong index or
transposed operand in oracle/ fails one of them.

  * the ten masks against the reference's lambdas, restated verbatim from
    extra_bench.py:41,56-61, and against closed-form visible-pair counts;
  * every softmax variant against torch's scaled_dot_product_attention
    (an independent implementation), in float64;
  * closed forms (causal row 0, constant V, q = 0 for softmax/sigmoid/ReLU);
  * degenerate-parameter invariants;
  * a float64 loop-level brute force on tiny shapes;
  * the reference's own bf16 gate (rel < 3e-2, synth10.py:173-184) between the
    fp32 oracle and the restated bf16 eager path;
  * a planted mistake (the masked-before-sigmoid reference of synth10.py:48)
    that the checks must reject.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle.brute import attention_brute
from oracle.generic import attention_ref, visible_mask
from oracle.variants import REF_OPS, eager_bf16, variant_ref

F64 = torch.float64


def _qkv(B, H, S, D, seed, dtype=torch.float64, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return tuple((torch.randn(B, H, S, D, generator=g) * scale).to(dtype) for _ in range(3))


# ---------------------------------------------------------------- masks ----
REFERENCE_LAMBDAS = {
    # extra_bench.py:41 (default), 56-61, verbatim semantics
    "causal": lambda i, j: j <= i,
    "bias_dilated": lambda i, j: (j <= i) & (((i - j) % 4) == 0),
    "bias_local": lambda i, j: (i - j).abs() < 256,
    "bias_block_diagonal": lambda i, j: ((i // 512) == (j // 512)) & (j <= i),
    "bias_prefix_lm": lambda i, j: (j <= i) | (j < 256),
    "bias_sliding_window": lambda i, j: (j <= i) & ((i - j) < 256),
}
GENERIC = {
    "causal": dict(causal=True),
    "bias_dilated": dict(causal=True, dilation=4),
    "bias_local": dict(causal=False, window=256),
    "bias_block_diagonal": dict(causal=True, block=512),
    "bias_prefix_lm": dict(causal=True, prefix=256),
    "bias_sliding_window": dict(causal=True, window=256),
}


@pytest.mark.parametrize("name", list(REFERENCE_LAMBDAS))
@pytest.mark.parametrize("S", [64, 300, 1024, 2048])
def test_masks_match_reference_lambdas(name, S):
    i, j = torch.arange(S).view(-1, 1), torch.arange(S).view(1, -1)
    ref = REFERENCE_LAMBDAS[name](i, j)
    assert torch.equal(visible_mask(S, **GENERIC[name]), ref)


def test_visible_counts_closed_forms():
    S, W = 2048, 256
    # sliding window: sum_i min(i+1, W)
    assert visible_mask(S, causal=True, window=W).sum().item() == W * S - W * (W - 1) // 2
    assert abs(visible_mask(S, causal=True, window=W).float().mean().item() - 0.1172) < 5e-5
    # causal: S(S+1)/2
    assert visible_mask(S, causal=True).sum().item() == S * (S + 1) // 2
    S = 4096
    # prefix-LM P: P*S + sum_{i>=P}(i+1-P)  (keys < P for all rows, plus causal keys >= P)
    P = 1024
    m = visible_mask(S, causal=True, prefix=P).sum().item()
    assert m == P * S + sum(i + 1 - P for i in range(P, S))
    assert abs(m / S ** 2 - 0.5313) < 5e-5
    # block-diagonal 256: non-causal S*256, causal (S/256) * 256*257/2
    assert visible_mask(S, causal=False, block=256).sum().item() == S * 256
    assert visible_mask(S, causal=True, block=256).sum().item() == (S // 256) * 256 * 257 // 2
    # local +-128 == |i-j| < 129: S*(2*129-1) - 2*sum_{k=1}^{128} k
    assert visible_mask(S, causal=False, window=129).sum().item() == S * 257 - 128 * 129
    # dilated 2 within a 1024 window: sum_i #{d in [0, min(i,1023)], d even}
    m = visible_mask(S, causal=True, dilation=2, window=1024).sum().item()
    assert m == sum(min(i, 1023) // 2 + 1 for i in range(S))


# ----------------------------------------------------- SDPA reductions -----
def _sdpa_masked(q, k, v, mask, scale):
    return F.scaled_dot_product_attention(q, k, v, attn_mask=mask, scale=scale)


@pytest.mark.parametrize("op", ["bias_sliding_window", "bias_local", "bias_dilated", "bias_block_diagonal",
                                "bias_prefix_lm"])
@pytest.mark.parametrize("D", [16, 64])
def test_mask_variants_equal_sdpa(op, D):
    S = 96
    params = {"bias_sliding_window": dict(window=17), "bias_local": dict(window=9),
              "bias_dilated": dict(dilation=3), "bias_block_diagonal": dict(block=20),
              "bias_prefix_lm": dict(prefix=13)}[op]
    q, k, v = _qkv(1, 2, S, D, 3)
    ref = variant_ref(op, q, k, v, dtype=F64, **params)
    kwargs = {"bias_sliding_window": dict(causal=True, window=17), "bias_local": dict(causal=False, window=9),
              "bias_dilated": dict(causal=True, dilation=3), "bias_block_diagonal": dict(causal=True, block=20),
              "bias_prefix_lm": dict(causal=True, prefix=13)}[op]
    mask = visible_mask(S, **kwargs)
    got = _sdpa_masked(q, k, v, mask, 1 / math.sqrt(D))
    assert torch.allclose(ref, got, atol=1e-10, rtol=1e-10)


def test_alibi_equals_sdpa_with_additive_bias():
    S, D, H = 80, 32, 3
    q, k, v = _qkv(1, H, S, D, 4)
    slopes = torch.tensor([0.5, 0.125, 2.0], dtype=F64)
    ref = variant_ref("bias_alibi", q, k, v, dtype=F64, slopes=slopes)
    i, j = torch.arange(S).view(-1, 1), torch.arange(S).view(1, -1)
    bias = slopes.view(H, 1, 1) * (j - i).to(F64)
    bias = bias.masked_fill(j > i, float("-inf")).unsqueeze(0)
    got = _sdpa_masked(q, k, v, bias, 1 / math.sqrt(D))
    assert torch.allclose(ref, got, atol=1e-10, rtol=1e-10)


@pytest.mark.parametrize("mode", ["mul", "div"])
def test_temperature_equals_sdpa_per_head_scale(mode):
    S, D, H = 70, 64, 4
    q, k, v = _qkv(1, H, S, D, 5)
    t = torch.tensor([0.5, 0.75, 1.25, 2.0], dtype=F64)
    ref = variant_ref("temp_perhead", q, k, v, dtype=F64, temperature=t, mode=mode)
    mask = visible_mask(S, causal=True)
    for h in range(H):
        sc = (t[h] if mode == "mul" else 1 / t[h]).item() / math.sqrt(D)
        got = _sdpa_masked(q[:, h:h + 1], k[:, h:h + 1], v[:, h:h + 1], mask, sc)
        assert torch.allclose(ref[:, h:h + 1], got, atol=1e-10, rtol=1e-10)


def test_softcap_equals_sdpa_with_logit_correction():
    # SDPA adds attn_mask to its own q.k*scale, so mask = softcap(s) - s (s from an
    # explicit fp64 matmul) plus -inf outside the causal mask reproduces softcap(s).
    S, D, cap = 64, 64, 5.0
    q, k, v = _qkv(1, 2, S, D, 6, scale=2.0)
    ref = variant_ref("softcap_gemma2", q, k, v, dtype=F64, softcap=cap)
    s = (q @ k.transpose(-2, -1)) / math.sqrt(D)
    corr = (torch.tanh(s / cap) * cap - s).masked_fill(~visible_mask(S, causal=True), float("-inf"))
    got = _sdpa_masked(q, k, v, corr, 1 / math.sqrt(D))
    assert torch.allclose(ref, got, atol=1e-9, rtol=1e-9)


# ----------------------------------------------------------- closed forms ---
SOFTMAX_OPS = ["temp_perhead", "bias_alibi", "bias_dilated", "bias_local", "bias_block_diagonal",
               "bias_prefix_lm", "softcap_gemma2", "bias_sliding_window"]


@pytest.mark.parametrize("op", [o for o in SOFTMAX_OPS if o not in ("bias_prefix_lm", "bias_local")])
def test_causal_row0_is_v0(op):
    q, k, v = _qkv(1, 2, 50, 32, 7)
    o = variant_ref(op, q, k, v, dtype=F64)
    assert torch.allclose(o[:, :, 0], v[:, :, 0], atol=1e-12)


@pytest.mark.parametrize("op", SOFTMAX_OPS)
def test_constant_v_gives_constant_o(op):
    q, k, _ = _qkv(1, 2, 64, 32, 8)
    v = torch.full((1, 2, 64, 32), 0.7, dtype=F64)
    o = variant_ref(op, q, k, v, dtype=F64)
    assert torch.allclose(o, torch.full_like(o, 0.7), atol=1e-12)


@pytest.mark.parametrize("op", ["bias_sliding_window", "bias_local", "bias_block_diagonal", "bias_prefix_lm",
                                "temp_perhead", "softcap_gemma2", "bias_dilated"])
def test_zero_q_gives_mean_of_visible_v(op):
    S, D = 60, 16
    _, k, v = _qkv(1, 1, S, D, 9)
    q = torch.zeros(1, 1, S, D, dtype=F64)
    params = {"bias_sliding_window": dict(window=7), "bias_local": dict(window=5), "bias_block_diagonal": dict(block=11),
              "bias_prefix_lm": dict(prefix=9), "bias_dilated": dict(dilation=3)}.get(op, {})
    gen = {"bias_sliding_window": dict(causal=True, window=7), "bias_local": dict(causal=False, window=5),
           "bias_block_diagonal": dict(causal=True, block=11), "bias_prefix_lm": dict(causal=True, prefix=9),
           "bias_dilated": dict(causal=True, dilation=3)}.get(op, dict(causal=True))
    o = variant_ref(op, q, k, v, dtype=F64, **params)
    m = visible_mask(S, **gen).to(F64)
    expect = (m @ v[0, 0]) / m.sum(-1, keepdim=True)
    assert torch.allclose(o[0, 0], expect, atol=1e-12)


def test_zero_q_sigmoid_and_relu():
    S, D = 40, 16
    _, k, v = _qkv(1, 1, S, D, 10)
    q = torch.zeros(1, 1, S, D, dtype=F64)
    m = visible_mask(S, causal=True).to(F64)
    o = variant_ref("sigmoid_attn", q, k, v, dtype=F64, bias=-0.7, post_scale=0.5)
    sig = 1 / (1 + math.exp(0.7))
    assert torch.allclose(o[0, 0], sig * 0.5 * (m @ v[0, 0]), atol=1e-12)
    o = variant_ref("relu_attn", q, k, v, dtype=F64)
    assert torch.count_nonzero(o) == 0


def test_alibi_zero_q_geometric_weights():
    # q = 0: softmax over j <= i of slope*(j - i): weights proportional to exp(slope*(j-i))
    S, D = 30, 8
    _, k, v = _qkv(1, 1, S, D, 11)
    q = torch.zeros(1, 1, S, D, dtype=F64)
    slope = 0.3
    o = variant_ref("bias_alibi", q, k, v, dtype=F64, slopes=torch.tensor([slope], dtype=F64))
    for i in (0, 5, 29):
        w = torch.tensor([math.exp(slope * (j - i)) for j in range(i + 1)], dtype=F64)
        expect = (w / w.sum()) @ v[0, 0, : i + 1]
        assert torch.allclose(o[0, 0, i], expect, atol=1e-12)


# ------------------------------------------------------------ invariants ----
def test_degenerate_parameters():
    S, D = 100, 32
    q, k, v = _qkv(1, 2, S, D, 12)
    causal = variant_ref("bias_sliding_window", q, k, v, dtype=F64, window=10 ** 6)
    assert torch.allclose(causal, variant_ref("bias_block_diagonal", q, k, v, dtype=F64, block=4096), atol=1e-12)
    assert torch.allclose(causal, variant_ref("bias_prefix_lm", q, k, v, dtype=F64, prefix=0), atol=1e-12)
    assert torch.allclose(causal, variant_ref("bias_dilated", q, k, v, dtype=F64, dilation=1), atol=1e-12)
    assert torch.allclose(causal, variant_ref("bias_alibi", q, k, v, dtype=F64,
                                              slopes=torch.zeros(2, dtype=F64)), atol=1e-12)
    assert torch.allclose(causal, variant_ref("temp_perhead", q, k, v, dtype=F64,
                                              temperature=torch.ones(2, dtype=F64)), atol=1e-12)
    assert torch.allclose(causal, variant_ref("softcap_gemma2", q, k, v, dtype=F64, softcap=1e7), atol=1e-9)
    full = attention_ref(q, k, v, causal=False, dtype=F64)
    assert torch.allclose(full, variant_ref("bias_prefix_lm", q, k, v, dtype=F64, prefix=S), atol=1e-12)
    assert torch.allclose(full, variant_ref("bias_local", q, k, v, dtype=F64, window=S), atol=1e-12)


# ------------------------------------------------------------ brute force ---
BRUTE_CASES = [
    dict(norm="softmax", causal=True),
    dict(norm="softmax", causal=False, window=3),
    dict(norm="softmax", causal=True, window=4, dilation=2),
    dict(norm="softmax", causal=True, block=5, prefix=3),
    dict(norm="softmax", causal=True, alibi_slopes=[0.5, 0.1], softcap=2.0),
    dict(norm="softmax", causal=True, head_scale=[0.5, 3.0]),
    dict(norm="sigmoid", causal=True, bias=-1.0, post_scale=0.5),
    dict(norm="sigmoid", causal=False, softcap=3.0, alibi_slopes=[0.2, -0.1]),
    dict(norm="relu", causal=True, post_scale=0.25, window=5),
    dict(norm="relu", causal=False, block=4),
]


@pytest.mark.parametrize("kw", BRUTE_CASES, ids=lambda k: ",".join(f"{a}={b}" for a, b in k.items()))
def test_generic_oracle_vs_brute_force(kw):
    q, k, v = _qkv(1, 2, 13, 16, 13)
    ref = attention_ref(q, k, v, dtype=F64, **kw)
    brute = attention_brute(q.numpy(), k.numpy(), v.numpy(), **kw)
    np.testing.assert_allclose(ref.numpy(), brute, atol=1e-12, rtol=1e-12)


@pytest.mark.parametrize("op", list(REF_OPS))
def test_variant_oracle_vs_generic(op):
    # the variant restatements and the parameterised oracle agree at the reference defaults
    q, k, v = _qkv(1, 2, 600, 32, 14)
    H = 2
    gen = {
        "sigmoid_attn": dict(norm="sigmoid", causal=True),
        "relu_attn": dict(norm="relu", causal=True),
        "temp_perhead": dict(causal=True, head_scale=(0.5 + torch.arange(H, dtype=torch.bfloat16) / H).double()),
        "bias_alibi": dict(causal=True, alibi_slopes=torch.arange(1, H + 1, dtype=F64)),
        "bias_dilated": dict(causal=True, dilation=4),
        "bias_local": dict(causal=False, window=256),
        "bias_block_diagonal": dict(causal=True, block=512),
        "bias_prefix_lm": dict(causal=True, prefix=256),
        "softcap_gemma2": dict(causal=True, softcap=30.0),
        "bias_sliding_window": dict(causal=True, window=256),
    }[op]
    a = variant_ref(op, q, k, v, dtype=F64)
    b = attention_ref(q, k, v, dtype=F64, **gen)
    assert torch.allclose(a, b, atol=1e-11, rtol=1e-11)


# ------------------------------------------------- bf16 eager vs fp32 oracle
@pytest.mark.parametrize("op", list(REF_OPS))
def test_eager_bf16_passes_reference_gate(op):
    q, k, v = _qkv(1, 2, 256, 64, 15, dtype=torch.bfloat16)
    for sc in (1.0, 0.01):
        qq, kk, vv = q * sc, k * sc, v * sc
        r = variant_ref(op, qq, kk, vv)
        e = eager_bf16(op, qq, kk, vv).float()
        rel = ((r - e).abs().max() / (r.abs().max() + 1e-6)).item()
        assert rel < 3e-2, (op, sc, rel)


# ---------------------------------------------------------- planted bug -----
def test_planted_masked_before_sigmoid_is_rejected():
    # synth10.py:48 zeroed the masked scores BEFORE the sigmoid, giving masked keys
    # weight sigmoid(0) = 0.5.  The zero-q closed form and the oracle comparison
    # must both reject that form.
    S, D = 64, 16
    q, k, v = _qkv(1, 1, S, D, 16)
    ok = visible_mask(S, causal=True).to(F64)

    def buggy(q_, k_, v_):
        s = (q_ @ k_.transpose(-2, -1)) / math.sqrt(D)
        return torch.sigmoid(s * ok) @ v_

    good = variant_ref("sigmoid_attn", q, k, v, dtype=F64)
    rel = ((good - buggy(q, k, v)).abs().max() / good.abs().max()).item()
    assert rel > 0.3
    qz = torch.zeros_like(q)
    expect = 0.5 * (ok @ v[0, 0])
    assert torch.allclose(variant_ref("sigmoid_attn", qz, k, v, dtype=F64)[0, 0], expect, atol=1e-12)
    assert not torch.allclose(buggy(qz, k, v)[0, 0], expect, atol=1e-3)


@pytest.mark.parametrize("H,Hkv", [(4, 2), (6, 1), (8, 4)])
def test_grouped_query_oracle_equals_sdpa_gqa(H, Hkv):
    """The oracle's grouped-query path (query head h reads K/V head h // (H // H_kv))
    against torch's own GQA implementation (scaled_dot_product_attention, enable_gqa)."""
    g = torch.Generator().manual_seed(H * 31 + Hkv)
    q = torch.randn(2, H, 80, 32, generator=g, dtype=torch.float64)
    k, v = (torch.randn(2, Hkv, 80, 32, generator=g, dtype=torch.float64) for _ in range(2))
    for causal, window in ((True, 0), (True, 11), (False, 0)):
        mask = visible_mask(80, causal=causal, window=window)
        want = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, enable_gqa=True)
        got = attention_ref(q, k, v, causal=causal, window=window, dtype=torch.float64)
        torch.testing.assert_close(got, want, rtol=1e-10, atol=1e-10)
