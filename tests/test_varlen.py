"""Packed variable-length batches without a GPU: the host check of cu_seqlens,
the C ABI's handling of the new field, and the registered operators' fake
implementations and autograd graph on meta tensors."""
import ctypes

import pytest
import torch
from torch.fx.experimental.proxy_tensor import make_fx

import chia_proj_amd  # noqa: F401
from chia_proj_amd import _lib, attention_varlen, make_args
from chia_proj_amd.attention import check_cu_seqlens


def test_cu_seqlens_checks():
    assert check_cu_seqlens(torch.tensor([0, 5, 5, 12]), 12) == (3, 7)
    assert check_cu_seqlens(torch.tensor([0, 5, 12], dtype=torch.int32), 12, max_seqlen=100) == (2, 100)
    assert check_cu_seqlens(torch.tensor([0, 0]), 0) == (1, 0)
    for bad, total in (([1, 5], 5), ([0, 5, 3], 3), ([0, 5], 6), ([0], 0)):
        with pytest.raises(ValueError):
            check_cu_seqlens(torch.tensor(bad), total)
    with pytest.raises(ValueError, match="max_seqlen"):
        check_cu_seqlens(torch.tensor([0, 5, 12]), 12, max_seqlen=6)
    with pytest.raises(TypeError):
        check_cu_seqlens(torch.tensor([0.0, 4.0]), 4)


def test_abi_field_and_alignment(lib_built):
    # the two pointers replaced reserved words: the struct keeps its size
    # (kv_heads + 7 reserved int32 before them)
    assert ctypes.sizeof(_lib.AttnArgs) == _lib.AttnArgs.kv_heads.offset + 32
    assert _lib.AttnArgs.cu_seqlens.offset % 8 == 0 and _lib.AttnArgs.seq_order.offset % 8 == 0
    a = make_args(batch=2, heads=1, seqlen=64, head_dim=64)
    a.q = a.k = a.v = a.o = 0x1000
    for name in ("q_stride", "k_stride", "v_stride", "o_stride"):
        st = getattr(a, name)
        st[0], st[1], st[2] = 0, 64, 64
    a.cu_seqlens = 0x2002  # not 4-byte aligned: rejected before any launch
    assert lib_built.chia_attn_fwd(ctypes.byref(a), None) == -7
    a.cu_seqlens = 0x2000
    a.seq_order = 0x3001
    assert lib_built.chia_attn_fwd(ctypes.byref(a), None) == -7
    a.cu_seqlens = a.seq_order = None
    a.reserved0 = 1
    assert lib_built.chia_attn_fwd(ctypes.byref(a), None) == -8


def _meta(T, H, D, grad=True):
    return torch.randn(T, H, D, device="meta", dtype=torch.bfloat16, requires_grad=grad)


@pytest.mark.parametrize("norm,lse_shape", [("softmax", (300, 4)), ("relu", (0, 0))])
def test_fake_shapes(norm, lse_shape):
    q, k = _meta(300, 4, 64), _meta(300, 2, 64)
    cu = torch.tensor([0, 100, 300], dtype=torch.int32, device="meta")
    o, lse = torch.ops.chia_attn.fwd_varlen(q, k, k, cu, 200, norm, True, 0, 1, 0, 0, None, None, None, 0.0, 0.0,
                                            1.0)
    assert o.shape == q.shape and lse.shape == lse_shape and not lse.requires_grad


def test_autograd_graph_is_two_nodes():
    q, k, v = _meta(300, 4, 64), _meta(300, 2, 64), _meta(300, 2, 64)
    cu = torch.tensor([0, 100, 300], dtype=torch.int32, device="meta")
    do = torch.empty(300, 4, 64, device="meta", dtype=torch.bfloat16)

    def f(q, k, v, do):
        return torch.autograd.grad(attention_varlen(q, k, v, cu, 200, causal=True, window=50), (q, k, v), do)

    gm = make_fx(f)(q, k, v, do)
    names = [str(n.target) for n in gm.graph.nodes if n.op == "call_function"]
    assert sum("fwd_varlen" in n for n in names) == 1 and sum("bwd_varlen" in n for n in names) == 1


def test_checked_offsets_are_cached_per_tensor_version():
    from chia_proj_amd.attention import _cu_plan

    cu = torch.tensor([0, 5, 12])
    first = _cu_plan(cu, 12, None, "cpu")
    assert _cu_plan(cu, 12, None, "cpu") is first            # same tensor, unchanged: no second check
    assert first[:2] == (2, 7) and first[3].tolist() == [1, 0]  # longest sequence dispatched first
    cu[1] = 3                                                 # an in-place change bumps the version
    again = _cu_plan(cu, 12, None, "cpu")
    assert again is not first and again[1] == 9
    cu[1] = 13                                                # and is checked again
    with pytest.raises(ValueError):
        _cu_plan(cu, 12, None, "cpu")
