"""bias_dilated: Dilated causal attention: j <= i and (i-j) % dilation == 0 (and i-j < window if window > 0).

Drop-in for ``launch_kernel(q, k, v)`` of the reference's ``bias_dilated_BEST.py``
modules; semantics from extra_bench.py:56.  Extra keyword arguments default to the
reference's constants.
"""
from ..attention import attention
from ._spec import core_kwargs, heads_of

OP = "bias_dilated"


def launch_kernel(q, k, v, *, dilation: int = 4, window: int = 0, scale=None):
    """bf16 q, k, v [B, H, S, D] on the GPU -> new bf16 o of the same shape."""
    return attention(q, k, v, **core_kwargs(OP, heads_of(q), dilation=dilation, window=window, scale=scale))
