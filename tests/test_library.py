"""torch.library registration (chia_proj_amd/library.py), checked without a GPU:
the schemas, the fake (shape-only) implementations on meta tensors, and that
make_fx / torch.compile(fullgraph=True) see the forward and the registered
backward as single nodes."""
import pytest
import torch
from torch.fx.experimental.proxy_tensor import make_fx

import chia_proj_amd  # noqa: F401  (registers the operators)
from chia_proj_amd import attention

FWD_ARGS = ["q", "k", "v", "norm", "causal", "window", "dilation", "block", "prefix", "scale", "head_scale",
            "alibi_slopes", "softcap", "bias", "post_scale"]


def _meta(B, H, S, D, grad=True):
    return torch.randn(B, H, S, D, device="meta", dtype=torch.bfloat16, requires_grad=grad)


def test_schemas():
    fs = torch.ops.chia_attn.fwd.default._schema
    bs = torch.ops.chia_attn.bwd.default._schema
    assert [a.name for a in fs.arguments] == FWD_ARGS
    assert [a.name for a in bs.arguments] == ["do", "q", "k", "v", "o", "lse"] + FWD_ARGS[3:]
    assert len(fs.returns) == 2 and len(bs.returns) == 3
    assert not any(a.alias_info for a in fs.arguments)  # functional: mutates nothing


@pytest.mark.parametrize("norm,lse_shape", [("softmax", (2, 4, 100)), ("sigmoid", (0,)), ("relu", (0,))])
def test_fake_forward_shapes(norm, lse_shape):
    q, k = _meta(2, 4, 100, 64), _meta(2, 2, 100, 64)
    o, lse = torch.ops.chia_attn.fwd(q, k, k, norm, True, 0, 1, 0, 0, None, None, None, 0.0, 0.0, 1.0)
    assert o.shape == q.shape and o.dtype == torch.bfloat16 and o.is_contiguous()
    assert lse.shape == lse_shape and lse.dtype == torch.float32
    assert o.requires_grad and not lse.requires_grad  # lse is marked non-differentiable


def test_fake_backward_shapes_grouped_query():
    q, k, v = _meta(1, 8, 64, 128), _meta(1, 2, 64, 128), _meta(1, 2, 64, 128)
    do = torch.empty(q.shape, device="meta", dtype=torch.bfloat16)
    lse = torch.empty(1, 8, 64, device="meta", dtype=torch.float32)
    dq, dk, dv = torch.ops.chia_attn.bwd(do, q, k, v, q, lse, "softmax", True, 0, 1, 0, 0, None, None, None, 0.0,
                                         0.0, 1.0)
    assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == v.shape


def _count(gm, name):
    return sum(1 for n in gm.graph.nodes if n.op == "call_function" and name in str(n.target))


@pytest.mark.parametrize("kw", [dict(causal=True, window=33, head_scale=[1.0, 2.0]),
                                dict(norm="sigmoid", causal=False, bias=-2.0, alibi_slopes=[0.1, 0.2]),
                                dict(norm="relu", causal=True, post_scale=0.5, softcap=20.0)])
def test_make_fx_forward_and_backward_are_single_nodes(kw):
    def f(q, k, v, do):
        return torch.autograd.grad(attention(q, k, v, **kw), (q, k, v), do)

    q, k, v = _meta(1, 2, 128, 64), _meta(1, 2, 128, 64), _meta(1, 2, 128, 64)
    do = torch.empty(q.shape, device="meta", dtype=torch.bfloat16)
    gm = make_fx(f)(q, k, v, do)
    assert _count(gm, "chia_attn.fwd") == 1 and _count(gm, "chia_attn.bwd") == 1
    # the backward gets the forward's o and lse, not a recomputation
    bwd = next(n for n in gm.graph.nodes if "chia_attn.bwd" in str(n.target))
    assert bwd.args[6] == kw.get("norm", "softmax")


def test_torch_compile_fullgraph_on_meta():
    def f(q, k, v):
        return attention(q, k, v, causal=True, window=33, head_scale=[1.0, 2.0],
                         alibi_slopes=torch.tensor([0.1, 0.2]))

    cf = torch.compile(f, backend="aot_eager", fullgraph=True)
    q, k, v = _meta(1, 2, 128, 64), _meta(1, 1, 128, 64), _meta(1, 1, 128, 64)
    o = cf(q, k, v)
    assert o.shape == q.shape and o.requires_grad
    o.sum().backward()
    assert q.grad.shape == q.shape and k.grad.shape == k.shape
    with torch.no_grad():
        assert cf(q, k, v).shape == q.shape


def test_fp8_forward_fake_and_compile_on_meta():
    """chia_attn::fwd_fp8: bf16 output of q's shape from float8 inputs of either
    format, one node under make_fx."""
    for dt in (torch.float8_e4m3fn, torch.float8_e5m2):
        q = torch.empty(2, 4, 100, 64, device="meta", dtype=dt)
        k = torch.empty(2, 2, 100, 64, device="meta", dtype=dt)
        o = torch.ops.chia_attn.fwd_fp8(q, k, k, 0.5, 0.25, 1.0, "softmax", True, 0, 1, 0, 0, None, None, None,
                                        0.0, 0.0, 1.0)
        assert o.shape == q.shape and o.dtype == torch.bfloat16
    fn = lambda q, k: torch.ops.chia_attn.fwd_fp8(q, k, k, 1.0, 1.0, 1.0, "relu", False, 0, 1, 0, 0, None,  # noqa
                                                  None, None, 0.0, 0.0, 1.0)
    g = make_fx(fn, tracing_mode="fake")(q, k)
    calls = [n for n in g.graph.nodes if n.op == "call_function"]
    assert [str(n.target) for n in calls] == ["chia_attn.fwd_fp8.default"]
