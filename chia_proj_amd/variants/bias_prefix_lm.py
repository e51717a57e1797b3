"""bias_prefix_lm: Prefix-LM attention: j <= i or j < prefix (the prefix is bidirectional).

Drop-in for ``launch_kernel(q, k, v)`` of the reference's ``bias_prefix_lm_BEST.py``
modules; semantics from extra_bench.py:59.  Extra keyword arguments default to the
reference's constants.
"""
from ..attention import attention
from ._spec import core_kwargs, heads_of

OP = "bias_prefix_lm"


def launch_kernel(q, k, v, *, prefix: int = 256, scale=None):
    """bf16 q, k, v [B, H, S, D] on the GPU -> new bf16 o of the same shape."""
    return attention(q, k, v, **core_kwargs(OP, heads_of(q), prefix=prefix, scale=scale))
