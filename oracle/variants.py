"""The ten variants, restated from the reference's eager closures.  TEST INFRASTRUCTURE ONLY.

Every function follows ``build_refs(S)`` of extra_bench.py:32-62 (the canonical
S-parameterised references) with the sigmoid fixed as in sigmoid_fix.py:34-40,
and exposes the constants the reference bakes into its closures as keyword
arguments with the reference's values as defaults.  The masks are written in
the reference's own form (extra_bench.py:56-61), independently of the
interval form the product uses, so that a test comparing the two pins the
product's mask reduction.

Two numeric modes:
  * ``variant_ref(op, q, k, v, dtype=torch.float32)`` -- every step in fp32
    (or fp64): the north-star gate's reference.
  * ``eager_bf16(op, q, k, v)`` -- the reference's own bf16 eager path: the
    score rounded to bf16 (extra_bench.py:39), bf16 temperature (:35) and
    ALiBi bias (:49), softmax in fp32 (:42), p rounded to bf16 before p @ v
    (:45).  This is what bench.py times as the CPU baseline.
"""
from __future__ import annotations

import math
from typing import Callable, Optional

import torch
import torch.nn.functional as F


def _idx(S: int):
    """I() of extra_bench.py:34 (CPU)."""
    return torch.arange(S).view(-1, 1), torch.arange(S).view(1, -1)


def _temp(H: int, temperature, mode: str, eager: bool, dtype):
    """TEMP of extra_bench.py:35 unless given; mode 'div' divides instead."""
    if temperature is None:
        t = 0.5 + torch.arange(H, dtype=torch.bfloat16) / H
    else:
        t = torch.as_tensor(temperature).reshape(H)
        t = t.to(torch.bfloat16) if eager else t
    t = t.to(torch.bfloat16 if eager else dtype)
    if mode == "div":
        t = 1.0 / t
    elif mode != "mul":
        raise ValueError(mode)
    return t.view(1, H, 1, 1)


def _slopes(H: int, slopes, dtype):
    """SLOPE of extra_bench.py:36 unless given ('standard' = 2^(-8(h+1)/H))."""
    if slopes is None or (isinstance(slopes, str) and slopes == "reference"):
        s = torch.arange(1, H + 1, dtype=torch.float32)
    elif isinstance(slopes, str) and slopes == "standard":
        s = torch.tensor([2.0 ** (-8.0 * (h + 1) / H) for h in range(H)], dtype=torch.float64)
    else:
        s = torch.as_tensor(slopes, dtype=torch.float64).reshape(H)
    return s.to(dtype).view(1, H, 1, 1)


def _mk(q, k, v, *, mod: Optional[Callable] = None, maskfn: Optional[Callable] = None, norm: str = "softmax",
        scale=None, bias: float = 0.0, post_scale: float = 1.0, eager: bool = False,
        dtype=torch.float32) -> torch.Tensor:
    """mk() of extra_bench.py:37-46 on the CPU; fp32/fp64 unless eager."""
    B, H, S, D = q.shape
    SC = 1.0 / math.sqrt(D) if scale is None else float(scale)
    if eager:  # differentiable (torch autograd of the eager bf16 path is a calibration point for gradients)
        q, k, v = (t.cpu().to(torch.bfloat16) for t in (q, k, v))
    else:
        q, k, v = (t.detach().cpu().to(dtype) for t in (q, k, v))
    s = (q @ k.transpose(-2, -1)) * SC
    if mod is not None:
        s = mod(s)
    i, j = _idx(S)
    ok = maskfn(i, j) if maskfn else (j <= i)
    work = torch.float32 if eager else dtype
    if norm == "softmax":
        p = torch.softmax(s.masked_fill(~ok, float("-inf")).to(work), -1)
        p = torch.nan_to_num(p, nan=0.0)  # rows with no visible key -> 0
    elif norm == "sigmoid":
        p = torch.sigmoid(s.to(work) + bias) * ok.to(work) * post_scale
    elif norm == "relu":
        p = F.relu(s.to(work)) * ok.to(work) * post_scale
    else:
        raise ValueError(norm)
    if eager:
        return p.to(torch.bfloat16) @ v
    return p @ v


def _causal_or_all(causal: bool):
    return (lambda i, j: j <= i) if causal else (lambda i, j: torch.ones(i.shape[0], j.shape[1], dtype=torch.bool))


def sigmoid_attn(q, k, v, *, causal=True, bias=0.0, post_scale=1.0, scale=None, eager=False, dtype=torch.float32):
    # sigmoid_fix.py:34-40: sigmoid first, then zero the masked positions
    return _mk(q, k, v, maskfn=_causal_or_all(causal), norm="sigmoid", bias=bias, post_scale=post_scale,
               scale=scale, eager=eager, dtype=dtype)


def relu_attn(q, k, v, *, causal=True, post_scale=1.0, scale=None, eager=False, dtype=torch.float32):
    # extra_bench.py:44,53
    return _mk(q, k, v, maskfn=_causal_or_all(causal), norm="relu", post_scale=post_scale, scale=scale,
               eager=eager, dtype=dtype)


def temp_perhead(q, k, v, *, temperature=None, mode="mul", causal=True, scale=None, eager=False,
                 dtype=torch.float32):
    # extra_bench.py:35,54: s * TEMP
    t = _temp(q.shape[1], temperature, mode, eager, dtype)
    return _mk(q, k, v, mod=lambda s: s * t, maskfn=_causal_or_all(causal), scale=scale, eager=eager, dtype=dtype)


def bias_alibi(q, k, v, *, slopes=None, causal=True, scale=None, eager=False, dtype=torch.float32):
    # extra_bench.py:47-50: s + (SLOPE * (j - i)).to(DT), then causal softmax
    H, S = q.shape[1], q.shape[2]
    sl = _slopes(H, slopes, torch.float32 if eager else dtype)
    i, j = _idx(S)

    def mod(s):
        b = sl * (j - i).to(sl.dtype)
        return s + (b.to(torch.bfloat16) if eager else b)

    return _mk(q, k, v, mod=mod, maskfn=_causal_or_all(causal), scale=scale, eager=eager, dtype=dtype)


def bias_dilated(q, k, v, *, dilation=4, window=0, scale=None, eager=False, dtype=torch.float32):
    # extra_bench.py:56: (j<=i) & ((i-j) % 4 == 0); optional window (BASELINE config c4c)
    def maskfn(i, j):
        ok = (j <= i) & (((i - j) % dilation) == 0)
        return ok & ((i - j) < window) if window else ok

    return _mk(q, k, v, maskfn=maskfn, scale=scale, eager=eager, dtype=dtype)


def bias_local(q, k, v, *, window=256, scale=None, eager=False, dtype=torch.float32):
    # extra_bench.py:57: |i-j| < 256
    return _mk(q, k, v, maskfn=lambda i, j: (i - j).abs() < window, scale=scale, eager=eager, dtype=dtype)


def bias_block_diagonal(q, k, v, *, block=512, causal=True, scale=None, eager=False, dtype=torch.float32):
    # extra_bench.py:58: (i//512 == j//512) & (j<=i)
    def maskfn(i, j):
        ok = (i // block) == (j // block)
        return ok & (j <= i) if causal else ok

    return _mk(q, k, v, maskfn=maskfn, scale=scale, eager=eager, dtype=dtype)


def bias_prefix_lm(q, k, v, *, prefix=256, scale=None, eager=False, dtype=torch.float32):
    # extra_bench.py:59: (j<=i) | (j<256)
    return _mk(q, k, v, maskfn=lambda i, j: (j <= i) | (j < prefix), scale=scale, eager=eager, dtype=dtype)


def softcap_gemma2(q, k, v, *, softcap=30.0, causal=True, scale=None, eager=False, dtype=torch.float32):
    # extra_bench.py:60: tanh(s/30)*30 before the causal mask
    return _mk(q, k, v, mod=lambda s: torch.tanh(s / softcap) * softcap, maskfn=_causal_or_all(causal),
               scale=scale, eager=eager, dtype=dtype)


def bias_sliding_window(q, k, v, *, window=256, scale=None, eager=False, dtype=torch.float32):
    # extra_bench.py:61: (j<=i) & ((i-j) < 256)
    return _mk(q, k, v, maskfn=lambda i, j: (j <= i) & ((i - j) < window), scale=scale, eager=eager, dtype=dtype)


REF_OPS = {
    "sigmoid_attn": sigmoid_attn,
    "relu_attn": relu_attn,
    "temp_perhead": temp_perhead,
    "bias_alibi": bias_alibi,
    "bias_dilated": bias_dilated,
    "bias_local": bias_local,
    "bias_block_diagonal": bias_block_diagonal,
    "bias_prefix_lm": bias_prefix_lm,
    "softcap_gemma2": softcap_gemma2,
    "bias_sliding_window": bias_sliding_window,
}


def variant_ref(op: str, q, k, v, *, dtype=torch.float32, heads_per_chunk: int = 4, **params) -> torch.Tensor:
    """fp32 (or fp64) reference of variant `op`, computed a few heads at a time."""
    fn = REF_OPS[op]
    B, H = q.shape[:2]
    outs = []
    for b in range(B):
        row = []
        for h0 in range(0, H, heads_per_chunk):
            h1 = min(H, h0 + heads_per_chunk)
            p = resolve_head_params(op, H, params, h0, h1)
            row.append(fn(q[b:b + 1, h0:h1], k[b:b + 1, h0:h1], v[b:b + 1, h0:h1], dtype=dtype, **p))
        outs.append(torch.cat(row, dim=1))
    return torch.cat(outs, dim=0)


def eager_bf16(op: str, q, k, v, **params) -> torch.Tensor:
    """The reference's bf16 eager path for variant `op` (CPU)."""
    return REF_OPS[op](q, k, v, eager=True, **params)


def resolve_head_params(op: str, H: int, params: dict, h0: int, h1: int) -> dict:
    """`params` for heads [h0, h1) of an H-head problem, with the reference's
    per-head defaults (extra_bench.py:35-36) resolved for the full H first."""
    p = dict(params)
    if op == "temp_perhead":
        t = p.get("temperature")
        full = (0.5 + torch.arange(H, dtype=torch.bfloat16) / H).float() if t is None else torch.as_tensor(t).reshape(H)
        p["temperature"] = full[h0:h1]
    if op == "bias_alibi":
        p["slopes"] = _slopes(H, p.get("slopes"), torch.float64).reshape(H)[h0:h1]
    return p


def variant_ref_heads(op: str, q, k, v, heads, *, dtype=torch.float32, **params):
    """fp32 reference for selected (b, h) pairs: list of [S, D] tensors."""
    H = q.shape[1]
    outs = []
    for b, h in heads:
        p = resolve_head_params(op, H, params, h, h + 1)
        sl = slice(h, h + 1)
        outs.append(REF_OPS[op](q[b:b + 1, sl], k[b:b + 1, sl], v[b:b + 1, sl], dtype=dtype, **p)[0, 0])
    return outs
