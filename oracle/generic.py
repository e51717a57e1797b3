"""Parameterised attention reference (fp32 or fp64 torch, CPU).  TEST INFRASTRUCTURE ONLY.

Semantics follow the reference's eager closures (extra_bench.py:37-46):
  s = (q @ k^T) * scale                       extra_bench.py:39
  s = mod(s)                                  extra_bench.py:40 (temperature :54, softcap :60, ALiBi :49)
  ok = maskfn(i, j)                           extra_bench.py:41, masks :56-61
  softmax: softmax(s.masked_fill(~ok, -inf))  extra_bench.py:42
  sigmoid: sigmoid(s) * ok                    sigmoid_fix.py:37-39 (sigmoid BEFORE masking)
  relu:    relu(s) * ok                       extra_bench.py:44
  o = p @ v                                   extra_bench.py:45
but every step runs in fp32 (or fp64) instead of rounding s and p to bf16:
the north-star gate compares the bf16 kernel output with an fp32 reference.
A softmax row with no visible key returns 0 (the reference would return NaN).
"""
from __future__ import annotations

import math
from typing import Optional

import torch


def visible_mask(S: int, *, causal: bool = True, window: int = 0, dilation: int = 1, block: int = 0,
                 prefix: int = 0) -> torch.Tensor:
    """Boolean [S, S] mask, ok[i, j] = query i sees key j, written from the definitions."""
    i = torch.arange(S).view(-1, 1)
    j = torch.arange(S).view(1, -1)
    d = i - j
    ok = (d >= 0) if causal else torch.ones(S, S, dtype=torch.bool)
    if window:
        ok = ok & ((d < window) if causal else (d.abs() < window))
    if dilation and dilation > 1:
        ok = ok & ((d % dilation) == 0)
    if block:
        ok = ok & ((i // block) == (j // block))
    if prefix:
        ok = ok | (j < prefix)
    return ok


def attention_ref(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, norm: str = "softmax",
                  causal: bool = True, window: int = 0, dilation: int = 1, block: int = 0, prefix: int = 0,
                  scale: Optional[float] = None, head_scale=None, alibi_slopes=None, softcap: float = 0.0,
                  bias: float = 0.0, post_scale: float = 1.0, dtype: torch.dtype = torch.float32,
                  heads_per_chunk: int = 4) -> torch.Tensor:
    """Reference output [B, H, S, D] in `dtype` on the CPU for bf16 (or float) inputs."""
    B, H, S, D = q.shape
    sc = 1.0 / math.sqrt(D) if scale is None else float(scale)
    ok = visible_mask(S, causal=causal, window=window, dilation=dilation, block=block, prefix=prefix)
    rel = (torch.arange(S).view(1, -1) - torch.arange(S).view(-1, 1)).to(dtype)  # j - i
    hs = None if head_scale is None else torch.as_tensor(head_scale, dtype=dtype).reshape(H).cpu()
    sl = None if alibi_slopes is None else torch.as_tensor(alibi_slopes, dtype=dtype).reshape(H).cpu()
    qf, kf, vf = (t.detach().to("cpu", dtype) for t in (q, k, v))
    if kf.shape[1] != H:  # grouped-query / multi-query: query head h reads K/V head h // (H // H_kv)
        if H % kf.shape[1] or vf.shape != kf.shape:
            raise ValueError(f"K/V heads {kf.shape[1]} must divide query heads {H}")
        kf = kf.repeat_interleave(H // kf.shape[1], dim=1)
        vf = vf.repeat_interleave(H // vf.shape[1], dim=1)
    out = torch.empty(B, H, S, D, dtype=dtype)
    for b in range(B):
        for h0 in range(0, H, heads_per_chunk):
            h1 = min(H, h0 + heads_per_chunk)
            s = (qf[b, h0:h1] @ kf[b, h0:h1].transpose(-2, -1)) * sc
            if hs is not None:
                s = s * hs[h0:h1].view(-1, 1, 1)
            if sl is not None:
                s = s + sl[h0:h1].view(-1, 1, 1) * rel
            if softcap:
                s = torch.tanh(s / softcap) * softcap
            if norm == "softmax":
                s = s.masked_fill(~ok, float("-inf"))
                mx = s.amax(-1, keepdim=True)
                mx = torch.where(torch.isfinite(mx), mx, torch.zeros_like(mx))
                e = torch.exp(s - mx)
                den = e.sum(-1, keepdim=True)
                p = torch.where(den > 0, e / den.clamp_min(torch.finfo(dtype).tiny), torch.zeros_like(e))
            elif norm == "sigmoid":
                p = torch.sigmoid(s + bias) * ok.to(dtype) * post_scale
            elif norm == "relu":
                p = torch.relu(s) * ok.to(dtype) * post_scale
            else:
                raise ValueError(f"unknown norm {norm!r}")
            out[b, h0:h1] = p @ vf[b, h0:h1]
    return out
