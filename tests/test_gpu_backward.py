"""GPU parity of the backward (chia_attn_bwd through attention()'s autograd path)
against the CPU gradient oracle (oracle/grad.py: autograd of the fp32 forward).

Gate (per gradient tensor, relative to its largest reference magnitude m, floored
at 1e-3 of the largest of the case's three gradients so an exactly-zero gradient,
e.g. dq of a row that sees one key, is compared on that scale):
max |g - ref| <= GRAD_MAX * m and mean |g - ref| <= GRAD_MEAN * m.  The kernel
takes bf16 inputs, computes in fp32 and rounds P and dS to bf16 for the MFMAs;
the thresholds sit above the error of the reference's own bf16 eager path
differentiated by torch (measured by test_error_vs_eager_bf16_backward).
"""
import pytest
import torch

import oracle
from oracle.grad import attention_grad_ref
from chia_proj_amd import OPS, attention, core_kwargs

pytestmark = pytest.mark.gpu

DEV = "cuda"
GRAD_MAX = 1e-2
GRAD_MEAN = 1e-3


def _say(msg):
    print(msg, flush=True)


def _grad_stats(got, ref, floor=0.0):
    err = (got.float().cpu() - ref).abs()
    m = max(ref.abs().max().item(), floor, 1e-30)
    return {"max_rel": err.max().item() / m, "mean_rel": err.mean().item() / m, "ref_max": ref.abs().max().item()}


def _check(name, grads, refs):
    floor = 1e-3 * max(r.abs().max().item() for r in refs)
    for label, g, r in zip(("dq", "dk", "dv"), grads, refs):
        st = _grad_stats(g, r, floor)
        assert torch.isfinite(g.float()).all(), (name, label)
        assert st["max_rel"] <= GRAD_MAX and st["mean_rel"] <= GRAD_MEAN, (name, label, st)


def _run(q, k, v, do, fn):
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    o = fn(qg, kg, vg)
    o.backward(do.to(DEV))
    torch.cuda.synchronize()
    return o, (qg.grad, kg.grad, vg.grad)


def _draw(B, H, Hkv, S, D, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    q = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16)
    k, v = (torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16) for _ in range(2))
    do = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16)
    return q, k, v, do


@pytest.mark.parametrize("op", list(OPS))
@pytest.mark.parametrize("D", [64, 128])
def test_variant_backward_reference_defaults(op, D):
    """Each of the ten variants (reference constants), B1 H4 S512."""
    _say(f"[bwd] defaults op={op} D={D}")
    q, k, v, do = _draw(1, 4, 4, 512, D, 2000 + D)
    _, grads = _run(q, k, v, do, lambda a, b, c: OPS[op](a, b, c))
    refs = attention_grad_ref(q, k, v, do, **core_kwargs(op, 4))
    _check(f"{op} D={D}", grads, refs)


EDGE = [
    # (name, B, H, Hkv, S, D, generic kwargs)
    ("S1_causal", 1, 2, 2, 1, 64, dict(causal=True)),
    ("S65_full", 1, 2, 2, 65, 64, dict(causal=False)),
    ("S200_window33", 2, 2, 2, 200, 64, dict(causal=True, window=33)),
    ("S257_local40_d128", 1, 2, 2, 257, 128, dict(causal=False, window=40)),
    ("S1000_dil3", 1, 2, 2, 1000, 64, dict(causal=True, dilation=3)),
    ("S777_block100", 1, 2, 2, 777, 64, dict(causal=True, block=100)),
    ("S600_prefix130", 1, 2, 2, 600, 64, dict(causal=True, prefix=130)),
    ("S512_alibi_softcap", 1, 2, 2, 512, 64, dict(causal=True, alibi_slopes=[0.5, 0.125], softcap=20.0)),
    ("S384_headscale_d128", 1, 2, 2, 384, 128, dict(causal=True, head_scale=[0.5, 2.0])),
    ("S500_sigmoid_window", 1, 2, 2, 500, 64, dict(norm="sigmoid", causal=True, window=100, bias=-1.5)),
    ("S333_relu_post", 1, 2, 2, 333, 64, dict(norm="relu", causal=False, post_scale=0.01)),
    ("S300_sigmoid_softcap_alibi", 1, 2, 2, 300, 128, dict(norm="sigmoid", causal=False, softcap=10.0,
                                                           alibi_slopes=[0.01, 0.02], bias=0.3)),
    ("gqa_causal_g2", 1, 4, 2, 640, 64, dict(causal=True)),
    ("mqa_window_g4", 2, 4, 1, 300, 64, dict(causal=True, window=70)),
    ("gqa_sigmoid_g2_d128", 1, 4, 2, 256, 128, dict(norm="sigmoid", causal=False, bias=-2.0)),
    # per-head scales that differ inside a K/V group: dK takes c1 per score
    ("gqa_headscale_g2", 1, 4, 2, 640, 64, dict(causal=True, head_scale=[0.5, 2.0, 1.0, 0.25])),
    ("gqa_headscale_sigmoid_d128", 1, 4, 2, 256, 128, dict(norm="sigmoid", causal=False, bias=-2.0,
                                                             head_scale=[1.0, 0.5, 2.0, 2.0])),
    ("mqa_headscale_relu_alibi", 1, 4, 1, 300, 64, dict(norm="relu", causal=True, post_scale=0.05,
                                                        head_scale=[1.0, 0.5, 0.25, 2.0],
                                                        alibi_slopes=[0.1, 0.05, 0.02, 0.01])),
]


@pytest.mark.parametrize("name,B,H,Hkv,S,D,kw", EDGE, ids=[e[0] for e in EDGE])
def test_backward_edge_cases(name, B, H, Hkv, S, D, kw):
    """Ragged lengths, every mask kind, modifiers, normalisers and grouped-query K/V."""
    _say(f"[bwd] edge {name}")
    q, k, v, do = _draw(B, H, Hkv, S, D, S * 13 + D + H)
    o, grads = _run(q, k, v, do, lambda a, b, c: attention(a, b, c, **kw))
    # the autograd forward is the plain forward
    assert torch.equal(o.detach(), attention(q.to(DEV), k.to(DEV), v.to(DEV), **kw))
    refs = attention_grad_ref(q, k, v, do, **kw)
    _check(name, grads, refs)


def test_backward_causal_s2048_sampled_heads():
    """B2 H4 S2048 D64 causal softmax: the full kernel grid, two heads checked."""
    _say("[bwd] causal S2048")
    q, k, v, do = _draw(2, 4, 4, 2048, 64, 77)
    _, grads = _run(q, k, v, do, lambda a, b, c: attention(a, b, c, causal=True))
    for b, h in ((0, 0), (1, 3)):
        refs = attention_grad_ref(q[b:b + 1, h:h + 1], k[b:b + 1, h:h + 1], v[b:b + 1, h:h + 1],
                                  do[b:b + 1, h:h + 1], causal=True)
        _check(f"S2048 b={b} h={h}", [g[b:b + 1, h:h + 1] for g in grads], refs)


def test_backward_is_deterministic():
    """No atomics: two backward passes give identical gradients."""
    q, k, v, do = _draw(1, 4, 2, 700, 64, 5)
    _, g1 = _run(q, k, v, do, lambda a, b, c: attention(a, b, c, causal=True, window=300))
    _, g2 = _run(q, k, v, do, lambda a, b, c: attention(a, b, c, causal=True, window=300))
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)


@pytest.mark.parametrize("op", ["bias_sliding_window", "temp_perhead", "softcap_gemma2", "sigmoid_attn"])
def test_error_vs_eager_bf16_backward(op):
    """The kernel's gradient error against the reference's bf16 eager path
    differentiated by torch, both measured against the fp32 oracle (printed)."""
    q, k, v, do = _draw(1, 2, 2, 384, 64, 31)
    _, grads = _run(q, k, v, do, lambda a, b, c: OPS[op](a, b, c))
    kw = core_kwargs(op, 2)
    refs = attention_grad_ref(q, k, v, do, **kw)
    qe, ke, ve = (t.clone().requires_grad_(True) for t in (q, k, v))
    oracle.eager_bf16(op, qe, ke, ve, **oracle.resolve_head_params(op, 2, {}, 0, 2)).backward(do)
    for label, g, ge, r in zip(("dq", "dk", "dv"), grads, (qe.grad, ke.grad, ve.grad), refs):
        ours, eager = _grad_stats(g, r), _grad_stats(ge, r)
        _say(f"[bwd] {op} {label}: ours max {ours['max_rel']:.2e} mean {ours['mean_rel']:.2e} | "
             f"eager bf16 max {eager['max_rel']:.2e} mean {eager['mean_rel']:.2e}")
        assert ours["max_rel"] <= GRAD_MAX and ours["mean_rel"] <= GRAD_MEAN
