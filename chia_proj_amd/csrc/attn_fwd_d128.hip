// attn_fwd_d128.hip -- instantiations of the forward core for head_dim 128:
// {2, 4} wavefronts per workgroup x 3 normalisers x ALiBi on/off x softcap
// on/off.  Split by head dim so the two halves compile in parallel.
#include "attn_fwd_kernel.h"

namespace chia {

using KernelFn = void (*)(FwdParams);

template <int NW, int NORM, bool AL, bool SC>
static KernelFn inst() {
  return attn_fwd_kernel<128, NW, NORM, AL, SC>;
}

template <int NW>
static KernelFn pick(int norm, bool alibi, bool softcap) {
  static const KernelFn table[3][2][2] = {
      {{inst<NW, NORM_SOFTMAX, false, false>(), inst<NW, NORM_SOFTMAX, false, true>()},
       {inst<NW, NORM_SOFTMAX, true, false>(), inst<NW, NORM_SOFTMAX, true, true>()}},
      {{inst<NW, NORM_SIGMOID, false, false>(), inst<NW, NORM_SIGMOID, false, true>()},
       {inst<NW, NORM_SIGMOID, true, false>(), inst<NW, NORM_SIGMOID, true, true>()}},
      {{inst<NW, NORM_RELU, false, false>(), inst<NW, NORM_RELU, false, true>()},
       {inst<NW, NORM_RELU, true, false>(), inst<NW, NORM_RELU, true, true>()}},
  };
  return table[norm][alibi ? 1 : 0][softcap ? 1 : 0];
}

KernelFn select_kernel_d128(int waves, int norm, bool alibi, bool softcap) {
  return waves == 2 ? pick<2>(norm, alibi, softcap) : pick<4>(norm, alibi, softcap);
}

}  // namespace chia
