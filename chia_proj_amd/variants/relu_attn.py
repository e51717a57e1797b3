"""relu_attn: ReLU attention: p = relu(s) * visible * post_scale (no normalisation).

Drop-in for ``launch_kernel(q, k, v)`` of the reference's ``relu_attn_BEST.py``
modules; semantics from extra_bench.py:44.  Extra keyword arguments default to the
reference's constants.
"""
from ..attention import attention
from ._spec import core_kwargs, heads_of

OP = "relu_attn"


def launch_kernel(q, k, v, *, causal: bool = True, post_scale: float = 1.0, scale=None):
    """bf16 q, k, v [B, H, S, D] on the GPU -> new bf16 o of the same shape."""
    return attention(q, k, v, **core_kwargs(OP, heads_of(q), causal=causal, post_scale=post_scale, scale=scale))
