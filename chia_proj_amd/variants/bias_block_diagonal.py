"""bias_block_diagonal: Block-diagonal attention: i // block == j // block (and j <= i when causal).

Drop-in for ``launch_kernel(q, k, v)`` of the reference's ``bias_block_diagonal_BEST.py``
modules; semantics from extra_bench.py:58.  Extra keyword arguments default to the
reference's constants.
"""
from ..attention import attention
from ._spec import core_kwargs, heads_of

OP = "bias_block_diagonal"


def launch_kernel(q, k, v, *, block: int = 512, causal: bool = True, scale=None):
    """bf16 q, k, v [B, H, S, D] on the GPU -> new bf16 o of the same shape."""
    return attention(q, k, v, **core_kwargs(OP, heads_of(q), block=block, causal=causal, scale=scale))
