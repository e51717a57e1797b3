"""torch.library registration of the attention core: ``chia_attn::fwd`` and ``chia_attn::bwd``.

The reference's kernels are plain Python functions that launch on torch's
current stream (extra_bench.py:12,19); torch.compile traces into them and
breaks its graph at the launch.  Registered as custom operators with fake
(shape-only) implementations and an autograd formula, the core is one opaque
node to torch.compile, make_fx and AOTAutograd -- the "operators Inductor does
not cover" use of the reference's README.md:3-6 -- and gradients flow through
the registered backward.

  chia_attn::fwd(q, k, v, <mask and score parameters>) -> (o, lse)
      o: bf16 like q; lse: float32 [B, H, S] (natural log, softmax only; an
      empty [0] tensor for sigmoid / ReLU).  lse is not differentiable.
  chia_attn::bwd(do, q, k, v, o, lse, <parameters>) -> (dq, dk, dv)

Per-head vectors are optional float32 device tensors [H]; ``scale`` None
stands for the default 1 / sqrt(head_dim).  Both operators run
``chia_attn_fwd_lse`` / ``chia_attn_bwd`` of libchia_attn.so on torch's current
stream, and raise if the library is not built.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import Tensor

from . import _lib

NAMESPACE = "chia_attn"


def _params(norm, causal, window, dilation, block, prefix, scale, head_scale, alibi_slopes, softcap, bias,
            post_scale) -> dict:
    return dict(norm=norm, causal=causal, window=window, dilation=dilation, block=block, prefix=prefix,
                scale=scale, head_scale=head_scale, alibi_slopes=alibi_slopes,
                softcap=softcap, bias=bias, post_scale=post_scale)


@torch.library.custom_op(f"{NAMESPACE}::fwd", mutates_args=(), device_types="cuda")
def fwd(q: Tensor, k: Tensor, v: Tensor, norm: str, causal: bool, window: int, dilation: int, block: int,
        prefix: int, scale: Optional[float], head_scale: Optional[Tensor], alibi_slopes: Optional[Tensor],
        softcap: float, bias: float, post_scale: float) -> Tuple[Tensor, Tensor]:
    from .attention import _prepare

    p = _params(norm, causal, window, dilation, block, prefix, scale, head_scale, alibi_slopes, softcap, bias,
                post_scale)
    o = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)  # contiguous, as the fake
    # Every tensor _prepare returns (layout copies of q, k, v and the per-head
    # vectors) stays referenced until the launch is queued: a copy freed earlier
    # would hand its memory to lse while the struct still points at it.
    a, hs, sl, qkv, _o = _prepare(q, k, v, o, **p)
    B, H, S, _ = q.shape
    if norm == "softmax":
        lse = torch.empty(B, H, S, dtype=torch.float32, device=q.device)
    else:
        lse = torch.empty(0, dtype=torch.float32, device=q.device)
    with torch.cuda.device(q.device):
        _lib.fwd_lse(a, lse.data_ptr() if lse.numel() else 0, torch.cuda.current_stream(q.device).cuda_stream)
    del qkv, hs, sl  # queued: torch's allocator orders any reuse after the launch on this stream
    return o, lse


@fwd.register_fake
def _fwd_fake(q, k, v, norm, causal, window, dilation, block, prefix, scale, head_scale, alibi_slopes, softcap,
              bias, post_scale):
    torch._check(q.dim() == 4, lambda: "q must be 4-D [B, H, S, D]")
    B, H, S, _ = q.shape
    lse_shape = (B, H, S) if norm == "softmax" else (0,)
    return torch.empty_like(q, memory_format=torch.contiguous_format), q.new_empty(lse_shape, dtype=torch.float32)


@torch.library.custom_op(f"{NAMESPACE}::bwd", mutates_args=(), device_types="cuda")
def bwd(do: Tensor, q: Tensor, k: Tensor, v: Tensor, o: Tensor, lse: Tensor, norm: str, causal: bool, window: int,
        dilation: int, block: int, prefix: int, scale: Optional[float], head_scale: Optional[Tensor],
        alibi_slopes: Optional[Tensor], softcap: float, bias: float, post_scale: float
        ) -> Tuple[Tensor, Tensor, Tensor]:
    from .attention import run_backward

    p = _params(norm, causal, window, dilation, block, prefix, scale, head_scale, alibi_slopes, softcap, bias,
                post_scale)
    return run_backward(do, q, k, v, o, lse if lse.numel() else None, p)


@bwd.register_fake
def _bwd_fake(do, q, k, v, o, lse, norm, causal, window, dilation, block, prefix, scale, head_scale, alibi_slopes,
              softcap, bias, post_scale):
    return (torch.empty_like(q, memory_format=torch.contiguous_format),
            torch.empty_like(k, memory_format=torch.contiguous_format),
            torch.empty_like(v, memory_format=torch.contiguous_format))


def _setup_context(ctx, inputs, output):
    q, k, v, *rest = inputs
    o, lse = output
    ctx.rest = rest  # norm .. post_scale, schema order (per-head tensors included)
    ctx.save_for_backward(q, k, v, o, lse)
    ctx.mark_non_differentiable(lse)
    ctx.set_materialize_grads(False)  # no zero-filled gradient for the unused lse


def _backward(ctx, do, _dlse):
    q, k, v, o, lse = ctx.saved_tensors
    if do is None:
        return (None,) * (3 + len(ctx.rest))
    # traced (torch.compile, make_fx / AOTAutograd: a dispatch mode is active, or
    # fake / meta tensors): the registered operator, one node of the graph;
    # eager on the GPU: the same implementation without a second operator dispatch
    traced = (torch.compiler.is_compiling() or torch._C._len_torch_dispatch_stack() > 0
              or type(do) is not torch.Tensor or do.device.type != "cuda")
    if traced:
        dq, dk, dv = torch.ops.chia_attn.bwd(do, q, k, v, o, lse, *ctx.rest)
    else:
        from .attention import run_backward

        dq, dk, dv = run_backward(do, q, k, v, o, lse if lse.numel() else None, _params(*ctx.rest))
    return (dq, dk, dv) + (None,) * len(ctx.rest)


fwd.register_autograd(_backward, setup_context=_setup_context)


def call_fwd(q: Tensor, k: Tensor, v: Tensor, params: dict) -> Tuple[Tensor, Tensor]:
    """torch.ops.chia_attn.fwd with attention()'s keyword parameters (per-head
    vectors already float32 device tensors or None; scale None = default)."""
    return torch.ops.chia_attn.fwd(q, k, v, params["norm"], bool(params["causal"]), int(params["window"] or 0),
                                   int(params["dilation"] or 1), int(params["block"] or 0),
                                   int(params["prefix"] or 0),
                                   None if params["scale"] is None else float(params["scale"]),
                                   params["head_scale"], params["alibi_slopes"], float(params["softcap"] or 0.0),
                                   float(params["bias"]), float(params["post_scale"]))


# ---- packed variable-length batches ------------------------------------------------
#   chia_attn::fwd_varlen(q, k, v, cu_seqlens, max_seqlen, <parameters>) -> (o, lse)
#       q, o [T, H, D]; k, v [T, H_kv, D]; lse float32 [T, H] (softmax) or [0]
#   chia_attn::bwd_varlen(do, q, k, v, o, lse, cu_seqlens, max_seqlen, <parameters>) -> (dq, dk, dv)
# max_seqlen <= 0: the longest sequence (read from cu_seqlens on the host).

def _max_len(max_seqlen: int):
    return None if max_seqlen <= 0 else max_seqlen


@torch.library.custom_op(f"{NAMESPACE}::fwd_varlen", mutates_args=(), device_types="cuda")
def fwd_varlen(q: Tensor, k: Tensor, v: Tensor, cu_seqlens: Tensor, max_seqlen: int, norm: str, causal: bool,
               window: int, dilation: int, block: int, prefix: int, scale: Optional[float],
               head_scale: Optional[Tensor], alibi_slopes: Optional[Tensor], softcap: float, bias: float,
               post_scale: float) -> Tuple[Tensor, Tensor]:
    from .attention import run_forward_varlen

    p = _params(norm, causal, window, dilation, block, prefix, scale, head_scale, alibi_slopes, softcap, bias,
                post_scale)
    return run_forward_varlen(q, k, v, cu_seqlens, _max_len(max_seqlen), p)


@fwd_varlen.register_fake
def _fwd_varlen_fake(q, k, v, cu_seqlens, max_seqlen, norm, causal, window, dilation, block, prefix, scale,
                     head_scale, alibi_slopes, softcap, bias, post_scale):
    torch._check(q.dim() == 3, lambda: "q must be 3-D [T, H, D]")
    T, H, _ = q.shape
    lse_shape = (T, H) if norm == "softmax" else (0, 0)
    return torch.empty_like(q, memory_format=torch.contiguous_format), q.new_empty(lse_shape, dtype=torch.float32)


@torch.library.custom_op(f"{NAMESPACE}::bwd_varlen", mutates_args=(), device_types="cuda")
def bwd_varlen(do: Tensor, q: Tensor, k: Tensor, v: Tensor, o: Tensor, lse: Tensor, cu_seqlens: Tensor,
               max_seqlen: int, norm: str, causal: bool, window: int, dilation: int, block: int, prefix: int,
               scale: Optional[float], head_scale: Optional[Tensor], alibi_slopes: Optional[Tensor], softcap: float,
               bias: float, post_scale: float) -> Tuple[Tensor, Tensor, Tensor]:
    from .attention import run_backward_varlen

    p = _params(norm, causal, window, dilation, block, prefix, scale, head_scale, alibi_slopes, softcap, bias,
                post_scale)
    return run_backward_varlen(do, q, k, v, o, lse, cu_seqlens, _max_len(max_seqlen), p)


@bwd_varlen.register_fake
def _bwd_varlen_fake(do, q, k, v, o, lse, cu_seqlens, max_seqlen, norm, causal, window, dilation, block, prefix,
                     scale, head_scale, alibi_slopes, softcap, bias, post_scale):
    return (torch.empty_like(q, memory_format=torch.contiguous_format),
            torch.empty_like(k, memory_format=torch.contiguous_format),
            torch.empty_like(v, memory_format=torch.contiguous_format))


def _setup_context_varlen(ctx, inputs, output):
    q, k, v, cu_seqlens, *rest = inputs
    o, lse = output
    ctx.rest = rest  # max_seqlen .. post_scale, schema order
    ctx.save_for_backward(q, k, v, o, lse, cu_seqlens)
    ctx.mark_non_differentiable(lse)
    ctx.set_materialize_grads(False)


def _backward_varlen(ctx, do, _dlse):
    q, k, v, o, lse, cu_seqlens = ctx.saved_tensors
    if do is None:
        return (None,) * (4 + len(ctx.rest))
    dq, dk, dv = torch.ops.chia_attn.bwd_varlen(do, q, k, v, o, lse, cu_seqlens, *ctx.rest)
    return (dq, dk, dv) + (None,) * (1 + len(ctx.rest))


fwd_varlen.register_autograd(_backward_varlen, setup_context=_setup_context_varlen)


def call_fwd_varlen(q: Tensor, k: Tensor, v: Tensor, cu_seqlens: Tensor, max_seqlen: Optional[int],
                    params: dict) -> Tuple[Tensor, Tensor]:
    """torch.ops.chia_attn.fwd_varlen with attention_varlen()'s keyword parameters."""
    return torch.ops.chia_attn.fwd_varlen(q, k, v, cu_seqlens, int(max_seqlen or 0), params["norm"],
                                          bool(params["causal"]), int(params["window"] or 0),
                                          int(params["dilation"] or 1), int(params["block"] or 0),
                                          int(params["prefix"] or 0),
                                          None if params["scale"] is None else float(params["scale"]),
                                          params["head_scale"], params["alibi_slopes"],
                                          float(params["softcap"] or 0.0), float(params["bias"]),
                                          float(params["post_scale"]))


# ---- FP8 forward -----------------------------------------------------------------

@torch.library.custom_op(f"{NAMESPACE}::fwd_fp8", mutates_args=(), device_types="cuda")
def fwd_fp8(q: Tensor, k: Tensor, v: Tensor, q_descale: float, k_descale: float, v_descale: float, norm: str,
            causal: bool, window: int, dilation: int, block: int, prefix: int, scale: Optional[float],
            head_scale: Optional[Tensor], alibi_slopes: Optional[Tensor], softcap: float, bias: float,
            post_scale: float) -> Tensor:
    from .attention import attention_fp8

    return attention_fp8(q, k, v, q_descale=q_descale, k_descale=k_descale, v_descale=v_descale,
                         **_params(norm, causal, window, dilation, block, prefix, scale, head_scale, alibi_slopes,
                                   softcap, bias, post_scale))


@fwd_fp8.register_fake
def _fwd_fp8_fake(q, k, v, q_descale, k_descale, v_descale, norm, causal, window, dilation, block, prefix, scale,
                  head_scale, alibi_slopes, softcap, bias, post_scale):
    torch._check(q.dim() == 4, lambda: "q must be 4-D [B, H, S, D]")
    return torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)


def call_fwd_fp8(q: Tensor, k: Tensor, v: Tensor, q_descale: float, k_descale: float, v_descale: float,
                 params: dict) -> Tensor:
    """torch.ops.chia_attn.fwd_fp8 with attention_fp8()'s keyword parameters (per-head
    vectors float32 device tensors or None; scale None = default)."""
    return torch.ops.chia_attn.fwd_fp8(q, k, v, float(q_descale), float(k_descale), float(v_descale),
                                       params["norm"], bool(params["causal"]), int(params["window"] or 0),
                                       int(params["dilation"] or 1), int(params["block"] or 0),
                                       int(params["prefix"] or 0),
                                       None if params["scale"] is None else float(params["scale"]),
                                       params["head_scale"], params["alibi_slopes"],
                                       float(params["softcap"] or 0.0), float(params["bias"]),
                                       float(params["post_scale"]))
