"""bias_sliding_window: Sliding-window causal attention: key j visible iff 0 <= i-j < window.

Drop-in for ``launch_kernel(q, k, v)`` of the reference's ``bias_sliding_window_BEST.py``
modules; semantics from extra_bench.py:61.  Extra keyword arguments default to the
reference's constants.
"""
from ..attention import attention
from ._spec import core_kwargs, heads_of

OP = "bias_sliding_window"


def launch_kernel(q, k, v, *, window: int = 256, scale=None):
    """bf16 q, k, v [B, H, S, D] on the GPU -> new bf16 o of the same shape."""
    return attention(q, k, v, **core_kwargs(OP, heads_of(q), window=window, scale=scale))
