"""float64 brute force over (i, j) for tiny shapes.  TEST INFRASTRUCTURE ONLY.

A third, loop-level statement of the semantics (mask predicate per pair,
score modifier per pair, normaliser per row) used to pin the vectorised
oracle on tiny inputs.  Follows extra_bench.py:37-46 and sigmoid_fix.py:34-40.
"""
from __future__ import annotations

import math

import numpy as np


def pair_visible(i: int, j: int, *, causal=True, window=0, dilation=1, block=0, prefix=0) -> bool:
    if prefix and j < prefix:
        return True
    d = i - j
    if causal and d < 0:
        return False
    if window and not (d < window if causal else abs(d) < window):
        return False
    if dilation > 1 and d % dilation != 0:
        return False
    if block and i // block != j // block:
        return False
    return True


def attention_brute(q, k, v, *, norm="softmax", causal=True, window=0, dilation=1, block=0, prefix=0,
                    scale=None, head_scale=None, alibi_slopes=None, softcap=0.0, bias=0.0,
                    post_scale=1.0) -> np.ndarray:
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, H, S, D = q.shape
    sc = 1.0 / math.sqrt(D) if scale is None else float(scale)
    out = np.zeros((B, H, S, D))
    for b in range(B):
        for h in range(H):
            hs = 1.0 if head_scale is None else float(head_scale[h])
            sl = 0.0 if alibi_slopes is None else float(alibi_slopes[h])
            for i in range(S):
                scores = []
                vis = []
                for j in range(S):
                    s = float(np.dot(q[b, h, i], k[b, h, j])) * sc * hs + sl * (j - i)
                    if softcap:
                        s = math.tanh(s / softcap) * softcap
                    scores.append(s)
                    vis.append(pair_visible(i, j, causal=causal, window=window, dilation=dilation, block=block,
                                            prefix=prefix))
                if norm == "softmax":
                    vs = [s for s, ok in zip(scores, vis) if ok]
                    if not vs:
                        continue
                    m = max(vs)
                    w = [math.exp(s - m) if ok else 0.0 for s, ok in zip(scores, vis)]
                    tot = sum(w)
                    p = [x / tot for x in w]
                elif norm == "sigmoid":
                    p = [post_scale / (1.0 + math.exp(-(s + bias))) if ok else 0.0 for s, ok in zip(scores, vis)]
                elif norm == "relu":
                    p = [post_scale * max(s, 0.0) if ok else 0.0 for s, ok in zip(scores, vis)]
                else:
                    raise ValueError(norm)
                out[b, h, i] = np.asarray(p) @ v[b, h]
    return out
