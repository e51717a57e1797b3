// attn_fwd_d64.hip -- instantiations of the forward core for head_dim 64
// (3 normalisers x ALiBi on/off x softcap on/off).  Split by head dim so the
// two halves compile in parallel.
#include "attn_fwd_kernel.h"

namespace chia {

using KernelFn = void (*)(FwdParams);

template <int NORM, bool AL, bool SC>
static KernelFn inst() {
  return attn_fwd_kernel<64, TileCfg<64>::QB, NORM, AL, SC>;
}

KernelFn select_kernel_d64(int norm, bool alibi, bool softcap) {
  static const KernelFn table[3][2][2] = {
      {{inst<NORM_SOFTMAX, false, false>(), inst<NORM_SOFTMAX, false, true>()},
       {inst<NORM_SOFTMAX, true, false>(), inst<NORM_SOFTMAX, true, true>()}},
      {{inst<NORM_SIGMOID, false, false>(), inst<NORM_SIGMOID, false, true>()},
       {inst<NORM_SIGMOID, true, false>(), inst<NORM_SIGMOID, true, true>()}},
      {{inst<NORM_RELU, false, false>(), inst<NORM_RELU, false, true>()},
       {inst<NORM_RELU, true, false>(), inst<NORM_RELU, true, true>()}},
  };
  return table[norm][alibi ? 1 : 0][softcap ? 1 : 0];
}

}  // namespace chia
