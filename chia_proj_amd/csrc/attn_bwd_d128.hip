// attn_bwd_d128.hip -- instantiations of the backward kernels for head_dim 128:
// 3 normalisers x ALiBi on/off x softcap on/off (dK/dV also with per-head c1).
#include "attn_bwd_kernel.h"

namespace chia {

template <int NORM, bool AL, bool SC>
static BwdKernels bwd_inst() {
  return BwdKernels{attn_bwd_dq_kernel<128, NORM, AL, SC>, attn_bwd_dkdv_kernel<128, NORM, AL, SC, false>,
                    attn_bwd_dkdv_kernel<128, NORM, AL, SC, true>};
}

BwdKernels select_bwd_kernels_d128(int norm, bool alibi, bool softcap) {
  static const BwdKernels table[3][2][2] = {
      {{bwd_inst<NORM_SOFTMAX, false, false>(), bwd_inst<NORM_SOFTMAX, false, true>()},
       {bwd_inst<NORM_SOFTMAX, true, false>(), bwd_inst<NORM_SOFTMAX, true, true>()}},
      {{bwd_inst<NORM_SIGMOID, false, false>(), bwd_inst<NORM_SIGMOID, false, true>()},
       {bwd_inst<NORM_SIGMOID, true, false>(), bwd_inst<NORM_SIGMOID, true, true>()}},
      {{bwd_inst<NORM_RELU, false, false>(), bwd_inst<NORM_RELU, false, true>()},
       {bwd_inst<NORM_RELU, true, false>(), bwd_inst<NORM_RELU, true, true>()}},
  };
  return table[norm][alibi ? 1 : 0][softcap ? 1 : 0];
}

}  // namespace chia
