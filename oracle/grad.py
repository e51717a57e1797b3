"""Gradients of the parameterised attention by autograd (CPU).  TEST INFRASTRUCTURE ONLY.

The reference is forward-only (README.md:223): the backward's semantics are
those of the forward formula of generic.py differentiated -- dL/dq, dL/dk,
dL/dv of L = sum(o * do), with the scale, per-head scale, ALiBi slopes,
softcap, sigmoid bias and post-scale as constants.  torch's autograd derives
the gradient here.  The one formula stated is _SoftmaxPV's backward, for
attention_grad_flash_model, a model of a fused backward's rounding; without
the rounding it must equal autograd (tests/test_oracle_grad.py).  A softmax row with no
visible key has o = 0 and no gradient.  K/V with fewer heads than Q
(grouped-query) are repeated per query head, so their gradients sum over the
group.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from .generic import visible_mask


class _SoftmaxPV(torch.autograd.Function):
    """o = P v with P = softmax(s) (rows without a visible key: 0), whose
    backward takes the softmax row term Delta_i = sum_j P_ij dP_ij in the form
    a fused kernel computes it, do_i . o_i, with o rounded to bf16 (the output
    the forward hands back) when round_o: dS = P * (dP - Delta), dv = P^T do.
    Without the rounding this is the softmax's own backward, which
    tests/test_oracle_grad.py checks against autograd."""

    @staticmethod
    def forward(ctx, s, row_any, v, round_o):
        p = torch.softmax(s, -1) * row_any.to(s.dtype)
        o = p @ v
        ctx.save_for_backward(p, v, o)
        ctx.round_o = round_o
        return o

    @staticmethod
    def backward(ctx, do):
        p, v, o = ctx.saved_tensors
        dp = do @ v.transpose(-2, -1)
        o_used = o.to(torch.bfloat16).to(o.dtype) if ctx.round_o else o
        delta = (do * o_used).sum(-1, keepdim=True)
        return p * (dp - delta), None, p.transpose(-2, -1) @ do, None


def attention_out_diff(q, k, v, *, norm: str = "softmax", causal: bool = True, window: int = 0, dilation: int = 1,
                       block: int = 0, prefix: int = 0, scale: Optional[float] = None, head_scale=None,
                       alibi_slopes=None, softcap: float = 0.0, bias: float = 0.0, post_scale: float = 1.0,
                       flash_delta: Optional[bool] = None):
    """The forward of generic.attention_ref as one differentiable expression (float tensors).

    flash_delta (softmax only): None differentiates softmax and P v by autograd;
    False / True route them through _SoftmaxPV, whose backward takes the row term
    from o exactly / from o rounded to bf16."""
    B, H, S, D = q.shape
    dtype = q.dtype
    sc = 1.0 / math.sqrt(D) if scale is None else float(scale)
    rep = H // k.shape[1]
    kr, vr = k.repeat_interleave(rep, 1), v.repeat_interleave(rep, 1)
    s = (q @ kr.transpose(-2, -1)) * sc
    if head_scale is not None:
        s = s * torch.as_tensor(head_scale, dtype=dtype).reshape(1, H, 1, 1)
    if alibi_slopes is not None:
        rel = (torch.arange(S).view(1, -1) - torch.arange(S).view(-1, 1)).to(dtype)  # j - i
        s = s + torch.as_tensor(alibi_slopes, dtype=dtype).reshape(1, H, 1, 1) * rel
    if softcap:
        s = torch.tanh(s / softcap) * softcap
    ok = visible_mask(S, causal=causal, window=window, dilation=dilation, block=block, prefix=prefix)
    if norm == "softmax":
        row_any = ok.any(-1, keepdim=True)
        s = torch.where(ok, s, torch.full_like(s, float("-inf")))
        s = torch.where(row_any, s, torch.zeros_like(s))  # rows with no key: finite, zeroed below
        if flash_delta is not None:
            return _SoftmaxPV.apply(s, row_any, vr, flash_delta)
        p = torch.softmax(s, -1) * row_any.to(dtype)
    elif norm == "sigmoid":
        p = torch.sigmoid(s + bias) * ok.to(dtype) * post_scale
    elif norm == "relu":
        p = torch.relu(s) * ok.to(dtype) * post_scale
    else:
        raise ValueError(f"unknown norm {norm!r}")
    return p @ vr


def attention_grad_ref(q, k, v, do, *, dtype: torch.dtype = torch.float32, **params):
    """(dq, dk, dv) in `dtype` on the CPU for bf16 (or float) q, k, v, do."""
    qf, kf, vf = (t.detach().to("cpu", dtype).requires_grad_(True) for t in (q, k, v))
    o = attention_out_diff(qf, kf, vf, **params)
    o.backward(do.detach().to("cpu", dtype))
    return qf.grad, kf.grad, vf.grad


def attention_grad_flash_model(q, k, v, do, *, dtype: torch.dtype = torch.float64, round_o: bool = True,
                               **params):
    """(dq, dk, dv) of the same forward for a softmax whose backward takes the row
    term Delta_i = do_i . o_i from the bf16 output o (round_o), as a fused
    backward that keeps only the bf16 o does; everything else in `dtype`.  The
    distance of these gradients from attention_grad_ref's is the error that
    rounding alone causes, which grows where dP - Delta cancels (a row that
    sees few keys of similar dP)."""
    qf, kf, vf = (t.detach().to("cpu", dtype).requires_grad_(True) for t in (q, k, v))
    o = attention_out_diff(qf, kf, vf, flash_delta=round_o, **params)
    o.backward(do.detach().to("cpu", dtype))
    return qf.grad, kf.grad, vf.grad
