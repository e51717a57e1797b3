"""chia_attn_bwd_noalloc through the C ABI: the backward with its row statistics
in the library's static per-GPU scratch, against chia_attn_bwd with a
caller-allocated workspace.  Both run the same kernels, so the gradients must
agree bit for bit; two calls in a row, the second on a smaller problem (the
scratch keeps the first call's contents), then a third of another head dim
and dilation.  A problem whose statistics exceed the scratch is refused on the
host before any launch."""
import ctypes

import pytest
import torch

from chia_proj_amd import _lib
from chia_proj_amd.attention import _op_forward, _prepare, run_backward

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(msg):
    print(msg, flush=True)


def _params(**kw):
    p = dict(norm="softmax", causal=True, window=0, dilation=1, block=0, prefix=0, scale=None, head_scale=None,
             alibi_slopes=None, softcap=0.0, bias=0.0, post_scale=1.0)
    p.update(kw)
    return p


def _noalloc_backward(do, q, k, v, o, lse, params):
    """dq, dk, dv by chia_attn_bwd_noalloc (no workspace passed)."""
    a, hs, sl, (q_, k_, v_), _ = _prepare(q, k, v, o, **params)
    dq, dk, dv = (torch.empty(t.shape, dtype=torch.bfloat16, device=t.device) for t in (q_, k_, v_))
    b = _lib.BwdArgs(dout=do.data_ptr(), dq=dq.data_ptr(), dk=dk.data_ptr(), dv=dv.data_ptr(),
                     lse=lse.data_ptr() if lse is not None else None, workspace=None, workspace_bytes=0)
    b.fwd = ctypes.pointer(a)
    for name, t in (("dout_stride", do), ("dq_stride", dq), ("dk_stride", dk), ("dv_stride", dv)):
        st = getattr(b, name)
        st[0], st[1], st[2] = t.stride(0), t.stride(1), t.stride(2)
    with torch.cuda.device(q_.device):
        _lib.bwd_noalloc(b, torch.cuda.current_stream(q_.device).cuda_stream)
    torch.cuda.synchronize()
    del q_, k_, v_, hs, sl
    return dq, dk, dv


CALLS = [
    # name, (B, H, Hkv, S, D), attention parameters; each problem smaller than the one before
    ("B2H4S1024_window300", (2, 4, 4, 1024, 64), _params(window=300)),
    ("B1H2S300_gqa", (1, 2, 1, 300, 64), _params()),
    ("B1H2S257_d128_dil3_alibi", (1, 2, 2, 257, 128), _params(dilation=3, alibi_slopes=[0.25, 0.5])),
]


def test_noalloc_backward_matches_workspace_backward():
    for name, (B, H, Hkv, S, D), params in CALLS:
        _say(f"[noalloc] {name}")
        g = torch.Generator("cpu").manual_seed(B * 1000 + S + D)
        q = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16).to(DEV)
        k, v = (torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16).to(DEV) for _ in range(2))
        do = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16).to(DEV)
        p = dict(params)
        if p["alibi_slopes"] is not None:
            p["alibi_slopes"] = torch.tensor(p["alibi_slopes"], dtype=torch.float32, device=DEV)
        o, lse = _op_forward(q, k, v, p)
        ref = run_backward(do, q, k, v, o, lse, p)
        got = _noalloc_backward(do, q, k, v, o, lse, p)
        torch.cuda.synchronize()
        for label, a, b in zip(("dq", "dk", "dv"), ref, got):
            assert bool(torch.isfinite(b).all()), (name, label)
            assert torch.equal(a, b), (name, label, (a.float() - b.float()).abs().max().item())


def test_noalloc_backward_without_statistics():
    """Sigmoid keeps no row statistics: the scratch is not touched, results still match."""
    _say("[noalloc] sigmoid")
    g = torch.Generator("cpu").manual_seed(5)
    q, k, v, do = (torch.randn(1, 2, 200, 64, generator=g).to(torch.bfloat16).to(DEV) for _ in range(4))
    p = _params(norm="sigmoid", causal=False, bias=-2.0)
    o, lse = _op_forward(q, k, v, p)
    ref = run_backward(do, q, k, v, o, None, p)
    got = _noalloc_backward(do, q, k, v, o, None, p)
    for a, b in zip(ref, got):
        assert torch.equal(a, b)


def test_noalloc_refuses_statistics_larger_than_the_scratch():
    """B16 H16 S8192 softmax needs 16 MiB of statistics: refused before any launch."""
    from chia_proj_amd.attention import make_args

    a = make_args(batch=16, heads=16, seqlen=8192, head_dim=64)
    assert _lib.bwd_workspace_size(a) > (8 << 20)
    a.q = a.k = a.v = a.o = 0x10000
    for name in ("q_stride", "k_stride", "v_stride", "o_stride"):
        st = getattr(a, name)
        st[0], st[1], st[2] = 16 * 8192 * 64, 8192 * 64, 64
    b = _lib.BwdArgs(fwd=ctypes.pointer(a), dout=0x20000, dq=0x30000, dk=0x40000, dv=0x50000, lse=0x60000)
    for name in ("dout_stride", "dq_stride", "dk_stride", "dv_stride"):
        st = getattr(b, name)
        st[0], st[1], st[2] = 16 * 8192 * 64, 8192 * 64, 64
    with pytest.raises(_lib.ChiaAttnError) as e:
        _lib.bwd_noalloc(b, 0)
    assert e.value.status == -10
