"""The ten attention variants, one module each, every one exposing
``launch_kernel(q, k, v, **params) -> o`` (the reference's drop-in protocol,
extra_bench.py:24-27).  ``OPS`` maps the reference's op names to those
functions."""
from . import (bias_alibi, bias_block_diagonal, bias_dilated, bias_local, bias_prefix_lm,
               bias_sliding_window, relu_attn, sigmoid_attn, softcap_gemma2, temp_perhead)
from ._spec import (OP_NAMES, core_kwargs, reference_alibi_slopes, reference_temperature,
                    standard_alibi_slopes)

_MODULES = {
    m.OP: m
    for m in (sigmoid_attn, relu_attn, temp_perhead, bias_alibi, bias_dilated, bias_local,
              bias_block_diagonal, bias_prefix_lm, softcap_gemma2, bias_sliding_window)
}
OPS = {name: _MODULES[name].launch_kernel for name in OP_NAMES}

__all__ = ["OPS", "OP_NAMES", "core_kwargs", "reference_alibi_slopes", "reference_temperature",
           "standard_alibi_slopes"]
