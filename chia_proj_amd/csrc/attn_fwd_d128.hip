// attn_fwd_d128.hip -- instantiations of the paired forward core for head_dim
// 128.  The dispatcher runs it only for sigmoid and ReLU on full rows of 2048
// keys or more without a score modifier, with 4 wavefronts per workgroup
// (every other head_dim 128 forward, softmax included, runs the one-block
// core, attn_fwd_q1_d128.hip).
#include "attn_fwd_kernel.h"

namespace chia {

using KernelFn = void (*)(FwdParams);

KernelFn select_kernel_d128(int norm) {
  if (norm == NORM_SIGMOID) return attn_fwd_kernel<128, 4, NORM_SIGMOID, false, false>;
  if (norm == NORM_RELU) return attn_fwd_kernel<128, 4, NORM_RELU, false, false>;
  return nullptr;  // softmax at head_dim 128 runs the one-block core
}

}  // namespace chia
