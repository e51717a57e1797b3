"""Variant definitions: reference defaults and the mapping to the generic core.

Each variant of the reference (extra_bench.py:51-62, sigmoid_fix.py:34-40) is
a fixed combination of mask, score modifier and normaliser.  ``to_kwargs``
turns a variant's public keyword arguments into the keyword arguments of
:func:`chia_proj_amd.attention.attention`; the defaults reproduce the
reference's constants (window 256, dilation 4, block 512, prefix 256,
ALiBi slope h+1, temperature 0.5+h/H, softcap 30, causal sigmoid/ReLU).
"""
from __future__ import annotations

import functools
from typing import Callable, Dict

import torch

OP_NAMES = (
    "sigmoid_attn",
    "relu_attn",
    "temp_perhead",
    "bias_alibi",
    "bias_dilated",
    "bias_local",
    "bias_block_diagonal",
    "bias_prefix_lm",
    "softcap_gemma2",
    "bias_sliding_window",
)


def reference_temperature(heads: int) -> torch.Tensor:
    """TEMP of extra_bench.py:35: (0.5 + arange(H)/H) evaluated in bf16, as float32."""
    return (0.5 + torch.arange(heads, dtype=torch.bfloat16) / heads).to(torch.float32)


def reference_alibi_slopes(heads: int) -> torch.Tensor:
    """SLOPE of extra_bench.py:36: h + 1."""
    return torch.arange(1, heads + 1, dtype=torch.float32)


def standard_alibi_slopes(heads: int) -> torch.Tensor:
    """Geometric ALiBi slopes m_h = 2^(-8(h+1)/H) (the BASELINE configuration)."""
    return torch.tensor([2.0 ** (-8.0 * (h + 1) / heads) for h in range(heads)], dtype=torch.float32)


@functools.lru_cache(maxsize=None)
def _preset_values(name: str, heads: int) -> tuple:
    """The float32 values of a per-head preset as a tuple of Python floats, built once per
    head count: a variant call with the default passes these host values, which the launch
    path keys by content, instead of building tensors on every call."""
    fn = {"temperature": reference_temperature, "alibi": reference_alibi_slopes,
          "standard": standard_alibi_slopes}[name]
    return tuple(fn(heads).tolist())


def _per_head(vals, heads: int, default: str):
    if vals is None:
        return _preset_values(default, heads)
    if isinstance(vals, str):
        if vals == "reference":
            return _preset_values(default, heads)
        if vals == "standard":
            return _preset_values("standard", heads)
        raise ValueError(f"unknown per-head preset {vals!r}")
    return vals


def kw_sliding_window(heads, *, window=256, scale=None):
    return dict(norm="softmax", causal=True, window=int(window), scale=scale)


def kw_local(heads, *, window=256, scale=None):
    return dict(norm="softmax", causal=False, window=int(window), scale=scale)


def kw_dilated(heads, *, dilation=4, window=0, scale=None):
    return dict(norm="softmax", causal=True, dilation=int(dilation), window=int(window or 0), scale=scale)


def kw_block_diagonal(heads, *, block=512, causal=True, scale=None):
    return dict(norm="softmax", causal=bool(causal), block=int(block), scale=scale)


def kw_prefix_lm(heads, *, prefix=256, scale=None):
    return dict(norm="softmax", causal=True, prefix=int(prefix), scale=scale)


def kw_alibi(heads, *, slopes=None, causal=True, scale=None):
    return dict(norm="softmax", causal=bool(causal), alibi_slopes=_per_head(slopes, heads, "alibi"), scale=scale)


def kw_softcap(heads, *, softcap=30.0, causal=True, scale=None):
    return dict(norm="softmax", causal=bool(causal), softcap=float(softcap), scale=scale)


def kw_temperature(heads, *, temperature=None, mode="mul", causal=True, scale=None):
    if mode not in ("mul", "div"):
        raise ValueError(f"mode must be 'mul' or 'div', got {mode!r}")
    if temperature is None or (isinstance(temperature, str) and temperature == "reference"):
        hs = _preset_values("temperature", heads) if mode == "mul" else _reciprocal_temperature(heads)
        return dict(norm="softmax", causal=bool(causal), head_scale=hs, scale=scale)
    t = _per_head(temperature, heads, "temperature")
    t = torch.as_tensor(t, dtype=torch.float32) if not isinstance(t, torch.Tensor) else t.to(torch.float32)
    hs = t if mode == "mul" else 1.0 / t
    return dict(norm="softmax", causal=bool(causal), head_scale=hs, scale=scale)


@functools.lru_cache(maxsize=None)
def _reciprocal_temperature(heads: int) -> tuple:
    """1 / t_h of the reference temperature, divided in float32 as for a tensor argument."""
    return tuple((1.0 / torch.tensor(_preset_values("temperature", heads), dtype=torch.float32)).tolist())


def kw_relu(heads, *, causal=True, post_scale=1.0, scale=None):
    return dict(norm="relu", causal=bool(causal), post_scale=float(post_scale), scale=scale)


def kw_sigmoid(heads, *, causal=True, bias=0.0, post_scale=1.0, scale=None):
    return dict(norm="sigmoid", causal=bool(causal), bias=float(bias), post_scale=float(post_scale), scale=scale)


TO_KWARGS: Dict[str, Callable] = {
    "bias_sliding_window": kw_sliding_window,
    "bias_local": kw_local,
    "bias_dilated": kw_dilated,
    "bias_block_diagonal": kw_block_diagonal,
    "bias_prefix_lm": kw_prefix_lm,
    "bias_alibi": kw_alibi,
    "softcap_gemma2": kw_softcap,
    "temp_perhead": kw_temperature,
    "relu_attn": kw_relu,
    "sigmoid_attn": kw_sigmoid,
}


def core_kwargs(op: str, heads: int, **params) -> dict:
    """Generic-core keyword arguments for variant `op` with `params`."""
    if op not in TO_KWARGS:
        raise KeyError(f"unknown variant {op!r}; known: {sorted(TO_KWARGS)}")
    return TO_KWARGS[op](heads, **params)


def heads_of(q) -> int:
    """Head count of a [B, H, S, D] tensor; 1 for anything else (the core then rejects it)."""
    shape = getattr(q, "shape", None)
    return int(shape[1]) if shape is not None and len(shape) == 4 else 1
