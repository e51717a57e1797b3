"""FP8 attention reference and the rounding model of the FP8 kernel (CPU).
TEST INFRASTRUCTURE ONLY.

The reference has no FP8 path (its kernels are bf16); the FP8 forward's
semantics are attention() of the DEQUANTISED inputs (stored e4m3 or e5m2 value
times its per-tensor descale), so `fp8_ref` is generic.attention_ref on those
values.  `fp8_emulated` adds the one rounding the FP8 path introduces besides
its inputs: the attention weights are scaled by 2^8 and rounded to e4m3 (torch's
float8_e4m3fn cast: round to nearest even), the row sum keeps the unrounded
weights (the kernels sum the rounded ones, so a row's dominant weight, which
this model keeps exact at 2^8, cancels between PV and the row sum; the
kernel's error is of the same order or below), o is rounded to bf16.  It
normalises with the exact row max where the
kernel uses the running max of the tiles seen so far, so it models the size of
the rounding error, not its bits; tests gate the kernel at a multiple of the
emulation's own error against fp8_ref.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from .generic import attention_ref, visible_mask


def dequant(x8: torch.Tensor, descale: float) -> torch.Tensor:
    return x8.to(torch.float32) * float(descale)


def fp8_ref(q8, k8, v8, q_descale=1.0, k_descale=1.0, v_descale=1.0, **params) -> torch.Tensor:
    """fp32 attention of the dequantised inputs (CPU)."""
    return attention_ref(dequant(q8.cpu(), q_descale), dequant(k8.cpu(), k_descale), dequant(v8.cpu(), v_descale),
                         **params)


def e4m3_round(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.float8_e4m3fn).to(x.dtype)


def fp8_emulated(q8, k8, v8, q_descale=1.0, k_descale=1.0, v_descale=1.0, *, norm: str = "softmax",
                 causal: bool = True, window: int = 0, dilation: int = 1, block: int = 0, prefix: int = 0,
                 scale: Optional[float] = None, head_scale=None, alibi_slopes=None, softcap: float = 0.0,
                 bias: float = 0.0, post_scale: float = 1.0) -> torch.Tensor:
    """The FP8 path's weight rounding applied to the exact computation (float64,
    bf16 output) for [B, H, S, D] inputs."""
    q, k, v = (dequant(t.cpu(), d).double() for t, d in ((q8, q_descale), (k8, k_descale), (v8, v_descale)))
    B, H, S, D = q.shape
    rep = H // k.shape[1]
    k, v = k.repeat_interleave(rep, 1), v.repeat_interleave(rep, 1)
    sc = 1.0 / math.sqrt(D) if scale is None else float(scale)
    s = (q @ k.transpose(-2, -1)) * sc
    if head_scale is not None:
        s = s * torch.as_tensor(head_scale, dtype=torch.float64).reshape(1, H, 1, 1)
    if alibi_slopes is not None:
        rel = (torch.arange(S).view(1, -1) - torch.arange(S).view(-1, 1)).double()
        s = s + torch.as_tensor(alibi_slopes, dtype=torch.float64).reshape(1, H, 1, 1) * rel
    if softcap:
        s = torch.tanh(s / softcap) * softcap
    ok = visible_mask(S, causal=causal, window=window, dilation=dilation, block=block, prefix=prefix)
    if norm == "softmax":
        s = s.masked_fill(~ok, float("-inf"))
        m = s.amax(-1, keepdim=True)
        m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
        w = torch.exp(s - m) * 256.0
        l = w.sum(-1, keepdim=True)
        o = (e4m3_round(w) @ v) / torch.where(l > 0, l, torch.ones_like(l))
    elif norm == "sigmoid":
        w = torch.sigmoid(s + bias) * 256.0 * ok
        o = (e4m3_round(w) @ v) * (post_scale / 256.0)
    elif norm == "relu":
        w = torch.relu(s).clamp(max=448.0) * ok
        o = (e4m3_round(w) @ v) * post_scale
    else:
        raise ValueError(f"unknown norm {norm!r}")
    return o.to(torch.bfloat16).to(torch.float32)
