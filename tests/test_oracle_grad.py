"""CPU pins of the gradient oracle (oracle/grad.py), which autograd derives from
a restatement of the forward.  The reference is forward-only, so nothing of its
own holds gradients; the pins are:
  * the differentiable forward equals the pinned forward oracle (attention_ref);
  * finite differences (torch.autograd.gradcheck, float64) for every kind of
    mask, score modifier and normaliser, and for grouped-query K/V;
  * torch's own scaled_dot_product_attention backward (an independent
    implementation) for softmax masks, with and without enable_gqa;
  * the fused-backward rounding model (attention_grad_flash_model): without
    its rounding it equals the autograd gradients in float64 (so its stated
    softmax backward is right), and its rounding moves dq and dk only.
"""
import pytest
import torch
import torch.nn.functional as F

from oracle.generic import attention_ref, visible_mask
from oracle.grad import attention_grad_flash_model, attention_grad_ref, attention_out_diff

CASES = [
    dict(causal=True),
    dict(causal=False),
    dict(causal=True, window=5),
    dict(causal=False, window=4),
    dict(causal=True, dilation=3),
    dict(causal=True, block=5),
    dict(causal=True, prefix=4),
    dict(causal=True, alibi_slopes=[0.5, 0.125]),
    dict(causal=True, head_scale=[0.5, 2.0]),
    dict(causal=True, softcap=1.5),
    dict(norm="sigmoid", causal=False, bias=-0.7, post_scale=0.5),
    dict(norm="sigmoid", causal=True, window=6, softcap=2.0, alibi_slopes=[0.2, -0.3]),
    dict(norm="relu", causal=True, post_scale=0.25),
    dict(norm="relu", causal=False, block=4, softcap=3.0),
]


def _inputs(H=2, Hkv=2, S=12, D=4, seed=0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, H, S, D, generator=g, dtype=torch.float64)
    k, v = (torch.randn(1, Hkv, S, D, generator=g, dtype=torch.float64) for _ in range(2))
    return q, k, v


@pytest.mark.parametrize("kw", CASES, ids=[str(c) for c in CASES])
def test_differentiable_forward_is_the_pinned_oracle(kw):
    q, k, v = _inputs(S=20, D=8)
    torch.testing.assert_close(attention_out_diff(q, k, v, **kw),
                               attention_ref(q, k, v, dtype=torch.float64, **kw), rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("kw", CASES, ids=[str(c) for c in CASES])
def test_gradient_matches_finite_differences(kw):
    q, k, v = (t.requires_grad_(True) for t in _inputs(seed=3))
    assert torch.autograd.gradcheck(lambda a, b, c: attention_out_diff(a, b, c, **kw), (q, k, v), eps=1e-6,
                                    atol=1e-6, rtol=1e-5)


def test_grouped_query_gradient_matches_finite_differences():
    q, k, v = (t.requires_grad_(True) for t in _inputs(H=4, Hkv=2, seed=5))
    assert torch.autograd.gradcheck(lambda a, b, c: attention_out_diff(a, b, c, causal=True, window=7), (q, k, v),
                                    eps=1e-6, atol=1e-6, rtol=1e-5)


@pytest.mark.parametrize("kw", [dict(causal=True), dict(causal=True, window=9), dict(causal=False, window=5),
                                dict(causal=True, block=7), dict(causal=True, prefix=6)])
@pytest.mark.parametrize("H,Hkv", [(2, 2), (4, 2), (4, 1)])
def test_softmax_gradient_equals_sdpa_backward(kw, H, Hkv):
    q, k, v = _inputs(H=H, Hkv=Hkv, S=40, D=16, seed=11)
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(12), dtype=torch.float64)
    got = attention_grad_ref(q, k, v, do, dtype=torch.float64, **kw)
    qs, ks, vs = (t.clone().requires_grad_(True) for t in (q, k, v))
    o = F.scaled_dot_product_attention(qs, ks, vs, attn_mask=visible_mask(40, **kw), enable_gqa=Hkv != H)
    o.backward(do)
    for g_got, g_want in zip(got, (qs.grad, ks.grad, vs.grad)):
        torch.testing.assert_close(g_got, g_want, rtol=1e-10, atol=1e-10)


SOFTMAX_CASES = [c for c in CASES if c.get("norm", "softmax") == "softmax"]


@pytest.mark.parametrize("kw", SOFTMAX_CASES, ids=[str(c) for c in SOFTMAX_CASES])
@pytest.mark.parametrize("H,Hkv", [(2, 2), (4, 1)])
def test_flash_model_without_rounding_is_autograd(kw, H, Hkv):
    q, k, v = _inputs(H=H, Hkv=Hkv, S=20, D=8, seed=11)
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(12), dtype=torch.float64)
    kw = {key: (val * (H // 2) if isinstance(val, list) else val) for key, val in kw.items()}  # per-head lists
    want = attention_grad_ref(q, k, v, do, dtype=torch.float64, **kw)
    got = attention_grad_flash_model(q, k, v, do, round_o=False, **kw)
    for g, w in zip(got, want):
        torch.testing.assert_close(g, w, rtol=1e-10, atol=1e-12)


def test_flash_model_rounding_moves_dq_dk_only():
    """The row term enters dS, so dq and dk move by at most the bf16 rounding of
    o times the size of do and the other operand; dv = P^T do does not move."""
    q, k, v = _inputs(H=2, Hkv=1, S=24, D=8, seed=13)
    do = torch.randn(q.shape, generator=torch.Generator().manual_seed(14), dtype=torch.float64)
    exact = attention_grad_ref(q, k, v, do, dtype=torch.float64, causal=True, window=2)
    model = attention_grad_flash_model(q, k, v, do, causal=True, window=2)
    torch.testing.assert_close(model[2], exact[2], rtol=0, atol=1e-12)
    for g, w in zip(model[:2], exact[:2]):
        moved = (g - w).abs().max().item()
        assert 0 < moved <= 2.0 ** -6 * w.abs().max().item()
