"""chia_proj_amd -- MI355X (gfx950) attention-variant forward library.

Ten attention variants (sliding-window, local, dilated, block-diagonal,
prefix-LM, ALiBi, Gemma-2 softcap, per-head temperature, ReLU, sigmoid) on one
hand-written HIP forward core, reached through the C ABI in
include/chia_attn.h.  ``OPS[name](q, k, v, **params)`` is the drop-in for the
reference's ``launch_kernel(q, k, v)``.
"""
from . import library  # registers torch.ops.chia_attn.fwd / bwd
from .attention import attention, attention_fp8, attention_fp8_varlen, attention_varlen, make_args, plan, quantize_fp8
from .variants import OP_NAMES, OPS, core_kwargs

__version__ = "0.1.0"

__all__ = ["attention", "attention_fp8", "attention_fp8_varlen", "quantize_fp8", "attention_varlen", "make_args", "plan", "library", "OPS", "OP_NAMES", "core_kwargs", "__version__"]
