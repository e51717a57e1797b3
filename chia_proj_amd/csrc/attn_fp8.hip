// attn_fp8.hip -- instantiations of the FP8 forward (attn_fp8_kernel.h).
#include "attn_fp8_kernel.h"

namespace chia {

template <int D, int FMT>
static Fp8KernelFn pick(int norm, bool alibi, bool softcap) {
#define CHIA_FP8(N, A, C) if (norm == N && alibi == A && softcap == C) return attn_fwd_fp8_kernel<D, N, A, C, FMT>;
#define CHIA_FP8_NORM(N) CHIA_FP8(N, false, false) CHIA_FP8(N, false, true) CHIA_FP8(N, true, false) CHIA_FP8(N, true, true)
  CHIA_FP8_NORM(NORM_SOFTMAX)
  CHIA_FP8_NORM(NORM_SIGMOID)
  CHIA_FP8_NORM(NORM_RELU)
#undef CHIA_FP8_NORM
#undef CHIA_FP8
  return nullptr;
}

Fp8KernelFn select_fp8_kernel(int head_dim, int format, int norm, bool alibi, bool softcap) {
  if (format == kFp8E5M2)
    return head_dim == 64 ? pick<64, kFp8E5M2>(norm, alibi, softcap) : pick<128, kFp8E5M2>(norm, alibi, softcap);
  return head_dim == 64 ? pick<64, kFp8E4M3>(norm, alibi, softcap) : pick<128, kFp8E4M3>(norm, alibi, softcap);
}

}  // namespace chia
