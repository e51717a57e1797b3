// attn_fwd_q1_d128.hip -- instantiations of the one-query-block-per-wavefront
// forward core (attn_fwd_q1_kernel.h) for head_dim 128: 3 normalisers x
// ALiBi on/off x softcap on/off, with one group of four wavefronts per
// workgroup or two, and softcap softmax against the fixed reference for caps
// up to 54 (attn_fwd_q1_d64.hip: head_dim 64).
#include "attn_fwd_q1_kernel.h"

namespace chia {

using KernelFn = void (*)(FwdParams);

template <int NORM, bool AL, bool SC, int NG = 1, bool CAPFIX = false>
static KernelFn inst_q1() {
  return attn_fwd_q1_kernel<128, NORM, AL, SC, NG, CAPFIX>;
}

KernelFn select_q1_kernel_d128(int norm, bool alibi, bool softcap, bool cap_fixed) {
  if (cap_fixed && norm == NORM_SOFTMAX && softcap)
    return alibi ? inst_q1<NORM_SOFTMAX, true, true, 1, true>() : inst_q1<NORM_SOFTMAX, false, true, 1, true>();
  static const KernelFn table[3][2][2] = {
      {{inst_q1<NORM_SOFTMAX, false, false>(), inst_q1<NORM_SOFTMAX, false, true>()},
       {inst_q1<NORM_SOFTMAX, true, false>(), inst_q1<NORM_SOFTMAX, true, true>()}},
      {{inst_q1<NORM_SIGMOID, false, false>(), inst_q1<NORM_SIGMOID, false, true>()},
       {inst_q1<NORM_SIGMOID, true, false>(), inst_q1<NORM_SIGMOID, true, true>()}},
      {{inst_q1<NORM_RELU, false, false>(), inst_q1<NORM_RELU, false, true>()},
       {inst_q1<NORM_RELU, true, false>(), inst_q1<NORM_RELU, true, true>()}},
  };
  return table[norm][alibi ? 1 : 0][softcap ? 1 : 0];
}

// Two groups per workgroup splitting each zigzag pair (small causal grids).
KernelFn select_q1_split_kernel_d128(int norm, bool alibi, bool softcap, bool cap_fixed) {
  if (cap_fixed && norm == NORM_SOFTMAX && softcap)
    return alibi ? inst_q1<NORM_SOFTMAX, true, true, 2, true>() : inst_q1<NORM_SOFTMAX, false, true, 2, true>();
  static const KernelFn table[3][2][2] = {
      {{inst_q1<NORM_SOFTMAX, false, false, 2>(), inst_q1<NORM_SOFTMAX, false, true, 2>()},
       {inst_q1<NORM_SOFTMAX, true, false, 2>(), inst_q1<NORM_SOFTMAX, true, true, 2>()}},
      {{inst_q1<NORM_SIGMOID, false, false, 2>(), inst_q1<NORM_SIGMOID, false, true, 2>()},
       {inst_q1<NORM_SIGMOID, true, false, 2>(), inst_q1<NORM_SIGMOID, true, true, 2>()}},
      {{inst_q1<NORM_RELU, false, false, 2>(), inst_q1<NORM_RELU, false, true, 2>()},
       {inst_q1<NORM_RELU, true, false, 2>(), inst_q1<NORM_RELU, true, true, 2>()}},
  };
  return table[norm][alibi ? 1 : 0][softcap ? 1 : 0];
}

}  // namespace chia
