"""temp_perhead: Per-head temperature causal attention: s * t_h (mode="mul", reference) or s / t_h (mode="div"). temperature=None is the reference's bf16 0.5 + h/H.

Drop-in for ``launch_kernel(q, k, v)`` of the reference's ``temp_perhead_BEST.py``
modules; semantics from extra_bench.py:35,54.  Extra keyword arguments default to the
reference's constants.
"""
from ..attention import attention
from ._spec import core_kwargs, heads_of

OP = "temp_perhead"


def launch_kernel(q, k, v, *, temperature=None, mode: str = "mul", causal: bool = True, scale=None):
    """bf16 q, k, v [B, H, S, D] on the GPU -> new bf16 o of the same shape."""
    return attention(q, k, v, **core_kwargs(OP, heads_of(q), temperature=temperature, mode=mode, causal=causal, scale=scale))
