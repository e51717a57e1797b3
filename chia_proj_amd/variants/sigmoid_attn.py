"""sigmoid_attn: Sigmoid attention: p = sigmoid(s + bias) * visible * post_scale; the sigmoid is taken before masking.

Drop-in for ``launch_kernel(q, k, v)`` of the reference's ``sigmoid_attn_BEST.py``
modules; semantics from sigmoid_fix.py:34-40.  Extra keyword arguments default to the
reference's constants.
"""
from ..attention import attention
from ._spec import core_kwargs, heads_of

OP = "sigmoid_attn"


def launch_kernel(q, k, v, *, causal: bool = True, bias: float = 0.0, post_scale: float = 1.0, scale=None):
    """bf16 q, k, v [B, H, S, D] on the GPU -> new bf16 o of the same shape."""
    return attention(q, k, v, **core_kwargs(OP, heads_of(q), causal=causal, bias=bias, post_scale=post_scale, scale=scale))
