// attn_fwd_q1_d64.hip -- instantiations of the one-query-block-per-wavefront
// forward core (attn_fwd_q1_kernel.h) for head_dim 64: 3 normalisers x
// ALiBi on/off x softcap on/off, and softcap softmax against the fixed
// reference for caps up to 54 (attn_fwd_q1_d128.hip: head_dim 128).
#include "attn_fwd_q1_kernel.h"

namespace chia {

using KernelFn = void (*)(FwdParams);

template <int NORM, bool AL, bool SC, bool CAPFIX = false>
static KernelFn inst_q1() {
  return attn_fwd_q1_kernel<64, NORM, AL, SC, 1, CAPFIX>;
}

KernelFn select_q1_kernel_d64(int norm, bool alibi, bool softcap, bool cap_fixed) {
  if (cap_fixed && norm == NORM_SOFTMAX && softcap)
    return alibi ? inst_q1<NORM_SOFTMAX, true, true, true>() : inst_q1<NORM_SOFTMAX, false, true, true>();
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

}  // namespace chia
