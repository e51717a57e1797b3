"""softcap_gemma2: Gemma-2 softcap causal attention: s = softcap * tanh(s / softcap), applied before the mask.

Drop-in for ``launch_kernel(q, k, v)`` of the reference's ``softcap_gemma2_BEST.py``
modules; semantics from extra_bench.py:60.  Extra keyword arguments default to the
reference's constants.
"""
from ..attention import attention
from ._spec import core_kwargs, heads_of

OP = "softcap_gemma2"


def launch_kernel(q, k, v, *, softcap: float = 30.0, causal: bool = True, scale=None):
    """bf16 q, k, v [B, H, S, D] on the GPU -> new bf16 o of the same shape."""
    return attention(q, k, v, **core_kwargs(OP, heads_of(q), softcap=softcap, causal=causal, scale=scale))
