// attn_fwd_d128.hip -- instantiations of the paired forward core for head_dim
// 128.  The dispatcher runs it only on full rows of 2048 keys or more without
// a score modifier, with 4 wavefronts per workgroup (every other head_dim
// 128 forward runs the one-block core, attn_fwd_q1_d128.hip): the three
// normalisers.
#include "attn_fwd_kernel.h"

namespace chia {

using KernelFn = void (*)(FwdParams);

KernelFn select_kernel_d128(int norm) {
  static const KernelFn table[3] = {attn_fwd_kernel<128, 4, NORM_SOFTMAX, false, false>,
                                    attn_fwd_kernel<128, 4, NORM_SIGMOID, false, false>,
                                    attn_fwd_kernel<128, 4, NORM_RELU, false, false>};
  return table[norm];
}

}  // namespace chia
