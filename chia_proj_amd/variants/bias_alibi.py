"""bias_alibi: ALiBi causal attention: s + slope_h * (j - i). slopes=None is the reference's h+1; "standard" gives 2^(-8(h+1)/H).

Drop-in for ``launch_kernel(q, k, v)`` of the reference's ``bias_alibi_BEST.py``
modules; semantics from extra_bench.py:36,47-50.  Extra keyword arguments default to the
reference's constants.
"""
from ..attention import attention
from ._spec import core_kwargs, heads_of

OP = "bias_alibi"


def launch_kernel(q, k, v, *, slopes=None, causal: bool = True, scale=None):
    """bf16 q, k, v [B, H, S, D] on the GPU -> new bf16 o of the same shape."""
    return attention(q, k, v, **core_kwargs(OP, heads_of(q), slopes=slopes, causal=causal, scale=scale))
