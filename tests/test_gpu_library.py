"""The registered operators on the GPU: torch.library.opcheck (schema, fake
implementation against the real one, autograd registration, AOT dispatch),
torch.compile(fullgraph=True) against eager, and the forward's lse output
against the oracle's log-sum-exp."""
import math

import pytest
import torch

import chia_proj_amd  # noqa: F401
from chia_proj_amd import attention, gate
from oracle.generic import visible_mask

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(msg):
    print(msg, flush=True)


def _qkv(B, H, Hkv, S, D, seed, grad=False):
    g = torch.Generator("cpu").manual_seed(seed)
    q = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16)
    k, v = (torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16) for _ in range(2))
    return tuple(t.to(DEV).requires_grad_(grad) for t in (q, k, v))


OPCHECK = [
    # name, (B, H, Hkv, S, D), positional parameters after q, k, v
    ("softmax_window", (1, 2, 2, 160, 64), ("softmax", True, 40, 1, 0, 0, None, None, None, 0.0, 0.0, 1.0)),
    ("sigmoid_alibi", (1, 2, 2, 96, 64), ("sigmoid", False, 0, 1, 0, 0, 0.2, None, "alibi", 0.0, -1.0, 1.0)),
    ("gqa_headscale_softcap_d128", (1, 4, 2, 130, 128),
     ("softmax", True, 0, 1, 0, 0, None, "head_scale", None, 15.0, 0.0, 1.0)),
    ("relu_prefix", (2, 2, 2, 100, 64), ("relu", True, 0, 1, 0, 17, None, None, None, 0.0, 0.0, 0.05)),
]


@pytest.mark.parametrize("name,shape,params", OPCHECK, ids=[c[0] for c in OPCHECK])
def test_opcheck_forward(name, shape, params):
    _say(f"[lib] opcheck {name}")
    q, k, v = _qkv(*shape, seed=len(name), grad=True)
    H = shape[1]
    p = list(params)
    for i, x in enumerate(p):
        if x == "alibi":
            p[i] = torch.linspace(0.05, 0.3, H, device=DEV)
        elif x == "head_scale":
            p[i] = torch.linspace(0.5, 1.5, H, device=DEV)
    torch.library.opcheck(torch.ops.chia_attn.fwd.default, (q, k, v, *p))


@pytest.mark.parametrize("norm", ["softmax", "sigmoid"])
def test_opcheck_backward(norm):
    _say(f"[lib] opcheck bwd {norm}")
    q, k, v = _qkv(1, 4, 2, 200, 64, seed=4)
    params = (norm, True, 64, 1, 0, 0, None, None, None, 0.0, 0.5, 1.0)
    o, lse = torch.ops.chia_attn.fwd(q, k, v, *params)
    do = torch.randn(q.shape, generator=torch.Generator("cpu").manual_seed(5)).to(torch.bfloat16).to(DEV)
    torch.library.opcheck(torch.ops.chia_attn.bwd.default, (do, q, k, v, o, lse, *params))


def test_compile_fullgraph_matches_eager():
    """A block (attention + output projection) under torch.compile(fullgraph) gives
    the eager outputs and gradients bit for bit: one opaque node each way."""
    _say("[lib] compile")
    q, k, v = _qkv(2, 4, 2, 256, 64, seed=9, grad=True)
    w = torch.randn(64, 64, device=DEV, dtype=torch.bfloat16, requires_grad=True)

    def block(q, k, v, w):
        o = attention(q, k, v, causal=True, window=100, head_scale=[0.5, 1.0, 1.5, 2.0])
        return o @ w

    outs = []
    for fn in (block, torch.compile(block, backend="aot_eager", fullgraph=True)):
        for t in (q, k, v, w):
            t.grad = None
        y = fn(q, k, v, w)
        y.float().square().sum().backward()
        outs.append((y.detach(), q.grad.clone(), k.grad.clone(), v.grad.clone(), w.grad.clone()))
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.parametrize("kw", [dict(causal=True), dict(causal=True, window=33, dilation=3),
                                dict(causal=False, block=50, alibi_slopes=[0.3, -0.2], softcap=10.0)])
def test_lse_output_matches_oracle(kw):
    """lse_i = log sum_j exp(s_ij) over visible keys (natural log, fp32), against
    a float64 CPU restatement of the score; a row with no visible key is -inf."""
    _say(f"[lib] lse {kw}")
    B, H, S, D = 1, 2, 300, 64
    q, k, v = _qkv(B, H, H, S, D, seed=3)
    params = dict(norm="softmax", window=0, dilation=1, block=0, prefix=0, scale=None, head_scale=None,
                  alibi_slopes=None, softcap=0.0, bias=0.0, post_scale=1.0)
    params.update(kw)
    from chia_proj_amd.attention import _op_forward
    _, lse = _op_forward(q, k, v, params)
    qd, kd = q.double().cpu(), k.double().cpu()
    s = (qd @ kd.transpose(-2, -1)) / math.sqrt(D)
    if params["alibi_slopes"] is not None:
        rel = (torch.arange(S).view(1, -1) - torch.arange(S).view(-1, 1)).double()
        s = s + torch.tensor(params["alibi_slopes"], dtype=torch.float64).view(1, H, 1, 1) * rel
    if params["softcap"]:
        s = torch.tanh(s / params["softcap"]) * params["softcap"]
    ok = visible_mask(S, causal=params["causal"], window=params["window"], dilation=params["dilation"],
                      block=params["block"], prefix=params["prefix"])
    ref = torch.logsumexp(s.masked_fill(~ok, float("-inf")), -1)
    got = lse.double().cpu()
    fin = torch.isfinite(ref)
    assert torch.equal(fin, torch.isfinite(got))
    assert (got[fin] - ref[fin]).abs().max().item() < 1e-3 * max(1.0, ref[fin].abs().max().item())


@pytest.mark.parametrize("dtype", [torch.float8_e4m3fn, torch.float8_e5m2])
def test_fp8_op_opcheck_and_compile(dtype):
    """chia_attn::fwd_fp8: opcheck's fake-against-real test, and torch.compile(fullgraph)
    of a block around it gives the eager bits."""
    from chia_proj_amd import attention_fp8, quantize_fp8
    _say(f"[lib] fp8 op {dtype}")
    q, k, v = _qkv(1, 4, 2, 192, 64, seed=21)
    (q8, qd), (k8, kd), (v8, vd) = (quantize_fp8(t, dtype=dtype) for t in (q, k, v))
    hs = torch.tensor([0.5, 1.0, 1.5, 2.0], device=DEV)
    # (opcheck's schema test perturbs the inputs with arithmetic torch has no float8 kernels for)
    torch.library.opcheck(torch.ops.chia_attn.fwd_fp8.default,
                          (q8, k8, v8, qd, kd, vd, "softmax", True, 50, 1, 0, 0, None, hs, None, 0.0, 0.0, 1.0),
                          test_utils=("test_faketensor",))
    direct = attention_fp8(q8, k8, v8, q_descale=qd, k_descale=kd, v_descale=vd, causal=True, window=50,
                           head_scale=hs)
    w = torch.randn(64, 64, device=DEV, dtype=torch.bfloat16)

    def block(q8, k8, v8, w):
        return torch.ops.chia_attn.fwd_fp8(q8, k8, v8, qd, kd, vd, "softmax", True, 50, 1, 0, 0, None, hs, None,
                                           0.0, 0.0, 1.0) @ w

    eager = block(q8, k8, v8, w)
    comp = torch.compile(block, backend="aot_eager", fullgraph=True)(q8, k8, v8, w)
    assert torch.equal(eager, comp)
    assert torch.equal(eager, direct @ w)


@pytest.mark.parametrize("norm", ["softmax", "sigmoid"])
def test_layout_copies_live_through_the_launch(norm):
    """q, k, v the kernel cannot read in place (unit stride on S, not on D: a
    [B, H, D, S] tensor viewed .mT) are copied to its layout inside the
    operators.  Each copy must stay allocated until its launch is queued, so
    that lse, dO, the gradients and the workspace allocated after it cannot take
    its memory.  The operator path (autograd) and the packed path are compared
    with the oracle: o, lse (against a float64 log-sum-exp) and the gradients."""
    from chia_proj_amd import attention_varlen
    from chia_proj_amd.attention import _op_forward
    from oracle.generic import attention_ref
    from oracle.grad import attention_grad_ref

    _say(f"[lib] layout copies {norm}")
    B, H, S, D = 2, 2, 320, 64
    g = torch.Generator("cpu").manual_seed(31)
    q, k, v, do = (torch.randn(B, H, D, S, generator=g).to(torch.bfloat16).mT for _ in range(4))
    assert q.stride(-1) != 1
    kw = dict(norm=norm, causal=True, window=150, bias=-1.0)
    params = dict(norm=norm, causal=True, window=150, dilation=1, block=0, prefix=0, scale=None, head_scale=None,
                  alibi_slopes=None, softcap=0.0, bias=-1.0, post_scale=1.0)
    qg, kg, vg = (t.to(DEV).requires_grad_(True) for t in (q, k, v))
    o, lse = _op_forward(qg, kg, vg, params)
    o.backward(do.to(DEV))
    torch.cuda.synchronize()
    ref = attention_ref(q, k, v, **kw)
    res = gate.north_star_gate(ref, o.detach().float().cpu(), scale_aware=norm != "softmax")
    assert res.ok, (res.status, res.stats)
    if norm == "softmax":
        s = (q.double() @ k.double().transpose(-2, -1)) / math.sqrt(D)
        ok = visible_mask(S, causal=True, window=150)
        lref = torch.logsumexp(s.masked_fill(~ok, float("-inf")), -1)
        assert (lse.double().cpu() - lref).abs().max().item() < 1e-3 * max(1.0, lref.abs().max().item())
    refs = attention_grad_ref(q, k, v, do, **kw)
    floor = 1e-3 * max(r.abs().max().item() for r in refs)
    for label, got, r in zip(("dq", "dk", "dv"), (qg.grad, kg.grad, vg.grad), refs):
        m = max(r.abs().max().item(), floor)
        err = (got.float().cpu() - r).abs()
        assert err.max().item() <= 1e-2 * m and err.mean().item() <= 1e-3 * m, (label, err.max().item(), m)

    # packed: [T, H, D] views with unit stride on T (copied inside), two sequences
    lens = [200, 120]
    T = sum(lens)
    qp, kp, vp, dop = (torch.randn(H, D, T, generator=g).to(torch.bfloat16).permute(2, 0, 1) for _ in range(4))
    assert qp.stride(-1) != 1
    cu = torch.tensor([0, lens[0], T], dtype=torch.int32)
    pg = [t.to(DEV).requires_grad_(True) for t in (qp, kp, vp)]
    op = attention_varlen(*pg, cu.to(DEV), **kw)
    op.backward(dop.to(DEV))
    torch.cuda.synchronize()
    for b in range(2):
        a0, a1 = int(cu[b]), int(cu[b + 1])
        seq = [t[a0:a1].transpose(0, 1).unsqueeze(0) for t in (qp, kp, vp, dop)]
        r = attention_ref(*seq[:3], **kw)[0]
        res = gate.north_star_gate(r, op[a0:a1].transpose(0, 1).detach().float().cpu(), scale_aware=norm != "softmax")
        assert res.ok, (b, res.status, res.stats)
        refs = attention_grad_ref(*seq, **kw)
        floor = 1e-3 * max(x.abs().max().item() for x in refs)
        for label, t, rr in zip(("dq", "dk", "dv"), pg, refs):
            got = t.grad[a0:a1].transpose(0, 1).unsqueeze(0).float().cpu()
            m = max(rr.abs().max().item(), floor)
            err = (got - rr).abs()
            assert err.max().item() <= 1e-2 * m and err.mean().item() <= 1e-3 * m, (b, label)
