"""FlexAttention semantics evaluated literally (CPU).  TEST INFRASTRUCTURE ONLY.

The reference writes its variants for torch's FlexAttention as a score
modifier and a mask predicate (extra_bench.py:85-99).  flex_ref applies the
callables themselves on the dense (q_idx, kv_idx) grid -- no fitting, no
parameters -- so a GPU result of chia_proj_amd.flex is checked against the
callables the user wrote:

    s  = (q . k) * scale                  (scale = 1 / sqrt(D) by default)
    s' = score_mod(s, b, h, q_idx, kv_idx)
    p  = softmax over kv_idx of s' where mask_mod(b, h, q_idx, kv_idx), 0 elsewhere
         (a row with no visible key gives 0)
         | sigmoid(s' + bias) * post_scale | relu(s') * post_scale, masked to 0
    o  = p @ v   (K / V heads repeated for grouped-query inputs)

The softmax definition is FlexAttention's; the sigmoid / ReLU normalisers are
the reference's own (sigmoid_fix.py:34-40, extra_bench.py:51-52), which
FlexAttention cannot express.  The callables are invoked on broadcast index
tensors ([S, 1] queries, [1, S] keys), as the predicates in the reference are.
"""
from __future__ import annotations

import math
from typing import Callable, Optional

import torch


def flex_ref(q, k, v, score_mod: Optional[Callable] = None, mask_mod: Optional[Callable] = None, *,
             scale: Optional[float] = None, norm: str = "softmax", bias: float = 0.0, post_scale: float = 1.0,
             dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Reference output [B, H, S, D] in `dtype` on the CPU."""
    B, H, S, D = q.shape
    rep = H // k.shape[1]
    sc = 1.0 / math.sqrt(D) if scale is None else float(scale)
    qi = torch.arange(S).view(S, 1)
    kj = torch.arange(S).view(1, S)
    out = torch.empty(B, H, S, D, dtype=dtype)
    for b in range(B):
        for h in range(H):
            qf = q[b, h].to(dtype)
            kf = k[b, h // rep].to(dtype)
            vf = v[b, h // rep].to(dtype)
            s = (qf @ kf.T) * sc
            bt, ht = torch.tensor(b), torch.tensor(h)
            if score_mod is not None:
                s = torch.as_tensor(score_mod(s, bt, ht, qi, kj)).to(dtype).expand(S, S)
            ok = (torch.as_tensor(mask_mod(bt, ht, qi, kj)).to(torch.bool).expand(S, S) if mask_mod is not None
                  else torch.ones(S, S, dtype=torch.bool))
            if norm == "softmax":
                row_any = ok.any(-1, keepdim=True)
                s = torch.where(ok, s, torch.full_like(s, float("-inf")))
                s = torch.where(row_any, s, torch.zeros_like(s))
                p = torch.softmax(s, -1) * row_any.to(dtype)
            elif norm == "sigmoid":
                p = torch.sigmoid(s + bias) * ok.to(dtype) * post_scale
            elif norm == "relu":
                p = torch.relu(s) * ok.to(dtype) * post_scale
            else:
                raise ValueError(f"unknown norm {norm!r}")
            out[b, h] = p @ vf
    return out
