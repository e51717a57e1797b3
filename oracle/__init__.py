"""oracle -- CPU restatement of the reference's attention-variant semantics.

TEST INFRASTRUCTURE ONLY.  Nothing in the product (chia_proj_amd/) imports
this package.  It is used by tests/ as the parity checker, by
__graft_entry__.smoke() as the checker of its one GPU call, and by bench.py's
cpu_baseline leg (timed as the reference's eager path on the host CPU, and as
the checker of the GPU output on the same bounded sample).

Modules
  variants.py  the ten variants written directly from the reference's eager
               closures (extra_bench.py:32-62, sigmoid_fix.py:34-40), in
               fp32/fp64 torch on the CPU, plus the reference's bf16 eager form.
  generic.py   the same semantics as one parameterised function (mask /
               score modifier / normaliser), used for edge cases the ten
               fixed variants do not reach.
  brute.py     float64 NumPy loops over (i, j) for tiny shapes.
  grad.py      the backward: autograd of generic.py's forward (dq, dk, dv).
  flex.py      FlexAttention's score_mod / mask_mod callables applied literally
               on the dense grid (the checker of chia_proj_amd.flex).

How each part is pinned (tests/test_oracle_*.py):
  * reductions to torch.nn.functional.scaled_dot_product_attention (an
    independent implementation) for every softmax variant;
  * closed forms (row 0 of a causal mask, constant V, q = 0 for softmax /
    sigmoid / ReLU);
  * degenerate-parameter invariants (window >= S is causal, block >= S is
    causal, prefix 0 is causal, dilation 1 is the plain mask, ...);
  * float64 brute force on tiny shapes;
  * the masks against the reference's own lambdas restated verbatim;
  * unmasked-fraction figures quoted from the reference's configuration
    analysis (11.72 % window-256 at S=2048, 53.13 % prefix-1024 at S=4096 ...).
  * grad.py: finite differences (gradcheck, float64) and SDPA's backward;
  * flex.py: equals generic.py on the reference's FlexAttention descriptions
    and on random mask parameter sets (the callables built from the
    definitions), and SDPA for plain causal softmax.
The reference holds no tensor-valued golden vectors (its results/ hold only
latencies and relative errors), so these checks are the pins.
"""
from .generic import attention_ref, visible_mask
from .variants import REF_OPS, eager_bf16, resolve_head_params, variant_ref, variant_ref_heads

__all__ = ["attention_ref", "visible_mask", "REF_OPS", "eager_bf16", "resolve_head_params", "variant_ref",
           "variant_ref_heads"]
