// attn_api.hip -- the C ABI (include/chia_attn.h): argument validation, the
// launch of the gfx950 core, and the host-only planning entry points.
//
// Reference boundary replaced: launch_kernel(q, k, v) -> o of
// kernels_gemini31propre_0018/<op>_BEST.py (e.g. bias_sliding_window_BEST.py:87-108).
// Unlike the reference (callee allocates o, shapes baked into each kernel),
// the caller passes o and every variant parameter explicitly.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstring>
#include <mutex>

#include "attn_fp8_kernel.h"
#include "chia_attn.h"

namespace chia {

using KernelFn = void (*)(FwdParams);
KernelFn select_kernel_d64(int waves, int norm, bool alibi, bool softcap);
KernelFn select_q1_kernel_d64(int norm, bool alibi, bool softcap, bool cap_fixed);
KernelFn select_kernel_d128(int norm);
KernelFn select_q1_kernel_d128(int norm, bool alibi, bool softcap, bool cap_fixed);
KernelFn select_q1_split_kernel_d128(int norm, bool alibi, bool softcap, bool cap_fixed);
BwdKernels select_bwd_kernels_d64(int norm, bool alibi, bool softcap);
BwdKernels select_bwd_kernels_d128(int norm, bool alibi, bool softcap);
Fp8KernelFn select_fp8_kernel(int head_dim, int format, int norm, bool alibi, bool softcap);

namespace {

constexpr int64_t kMaxSeq = (int64_t)1 << 28;
constexpr int64_t kMaxKvRowStride = (int64_t)1 << 25;  // elements between K/V rows the kernel steps over

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15u) == 0; }
bool stride_ok(const int64_t* s) { return s[0] % 8 == 0 && s[1] % 8 == 0 && s[2] % 8 == 0; }

int validate(const chia_attn_args* a, bool need_tensors) {
  if (!a) return CHIA_ATTN_ERR_NULL;
  if (a->struct_size != sizeof(chia_attn_args)) return CHIA_ATTN_ERR_STRUCT;
  if (need_tensors && (!a->q || !a->k || !a->v || !a->o)) return CHIA_ATTN_ERR_NULL;
  if (a->batch < 1 || a->heads < 1 || a->seqlen < 1 || a->seqlen >= kMaxSeq) return CHIA_ATTN_ERR_SHAPE;
  if (a->batch * a->heads > ((int64_t)1 << 24)) return CHIA_ATTN_ERR_SHAPE;
  if (a->head_dim != 64 && a->head_dim != 128) return CHIA_ATTN_ERR_HEAD_DIM;
  if (a->norm > CHIA_ATTN_NORM_RELU) return CHIA_ATTN_ERR_NORM;
  if (a->window < 0 || a->dilation < 1 || a->block < 0 || a->prefix < 0) return CHIA_ATTN_ERR_MASK;
  // A prefix seen by every query crosses the dilation residue classes the
  // kernel splits the problem into; the combination is rejected.
  if (a->dilation > 1 && a->prefix > 0) return CHIA_ATTN_ERR_MASK;
  if (!(a->scale > 0.f) || !std::isfinite(a->scale)) return CHIA_ATTN_ERR_SCALE;
  if (!(a->softcap >= 0.f) || !std::isfinite(a->softcap)) return CHIA_ATTN_ERR_SCALE;
  if (!std::isfinite(a->bias) || !std::isfinite(a->post_scale)) return CHIA_ATTN_ERR_SCALE;
  if (a->reserved0 != 0) return CHIA_ATTN_ERR_STRUCT;
  for (int i = 0; i < 2; ++i)
    if (a->reserved[i] != 0) return CHIA_ATTN_ERR_STRUCT;
  if (a->kv_heads < 0 || (a->kv_heads > 0 && a->heads % a->kv_heads != 0)) return CHIA_ATTN_ERR_SHAPE;
  if (need_tensors) {
    if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v) || !aligned16(a->o)) return CHIA_ATTN_ERR_ALIGN;
    if (!stride_ok(a->q_stride) || !stride_ok(a->k_stride) || !stride_ok(a->v_stride) || !stride_ok(a->o_stride))
      return CHIA_ATTN_ERR_ALIGN;
    if (((uintptr_t)a->head_scale & 3u) || ((uintptr_t)a->alibi_slopes & 3u) || ((uintptr_t)a->cu_seqlens & 3u) ||
        ((uintptr_t)a->seq_order & 3u))
      return CHIA_ATTN_ERR_ALIGN;
    // K/V tile loads address a tile's rows with 32-bit byte offsets from the
    // tile's first row: 64 rows x (seq stride x dilation) x 2 bytes < 2^32.
    for (const int64_t* st : {a->k_stride, a->v_stride})
      if (st[2] < 0 || st[2] * a->dilation >= kMaxKvRowStride) return CHIA_ATTN_ERR_SHAPE;
  }
  return CHIA_ATTN_OK;
}

// Packed sequences step through tokens with stride[2] from each sequence's
// first token; the batch stride is not used.
int64_t batch_stride(const chia_attn_args* a, const int64_t* st) { return a->cu_seqlens ? 0 : st[0]; }

MaskSpec spec_of(const chia_attn_args* a) {
  return make_mask_spec((int32_t)a->seqlen, a->causal ? 1 : 0, a->window, a->dilation, a->block, a->prefix);
}

constexpr int kCUs = 256;  // MI355X compute units

// Plain causal bands (no window, no block) make a row block's work grow with
// its position; such problems pair blocks (i, n-1-i) so every workgroup does
// the same work.
bool zigzag_of(const MaskSpec& m) { return m.lo >= 0 && m.hi >= kInf && m.blk == 0; }

// Score path of a forward call: the kernel instantiation's ALiBi / softcap
// switches.  The plain sigmoid kernel takes the bias as the factor
// 2^(-bias log2 e), which must be a normal float; a larger |bias| runs the
// general score path (the ALiBi kernel with null, i.e. zero, slopes).
struct ScorePath {
  bool alibi, softcap;
};
ScorePath score_path_of(const chia_attn_args* a) {
  ScorePath sp{a->alibi_slopes != nullptr, a->softcap > 0.f};
  if (a->norm == CHIA_ATTN_NORM_SIGMOID && !sp.alibi && !sp.softcap && !(std::fabs(-a->bias * kLog2e) <= 120.f))
    sp.alibi = true;
  return sp;
}

// Launch geometry shared by chia_attn_fwd and the planner.
struct Geometry {
  int waves;       // wavefronts per workgroup
  int rows;        // rows per row block (32 per wavefront)
  int n_pairs;     // workgroups per (b, h, residue 0): row-block pairs, or
                   // for the one-block core without pairing, row blocks
  int residues;
  int zigzag;
  bool q1;         // the one-block core (attn_fwd_q1_kernel.h)
  int groups;      // one-block core: groups of `waves` wavefronts per workgroup (2: a
                   // zigzag pair's steps split between two groups)
  bool rank;       // launch the units with the most keys first (rank_order)
  int64_t workgroups;
};

// The paired core: a workgroup owns two row blocks.
Geometry paired_geometry(const MaskSpec& m, int64_t batch, int64_t heads) {
  Geometry geo;
  geo.residues = num_residues(m);
  geo.zigzag = zigzag_of(m) ? 1 : 0;
  geo.q1 = false;
  geo.groups = 1;
  geo.rank = false;
  const int32_t s0 = residue_geom(m, 0).S;  // longest residue class
  // 4 wavefronts share each K/V tile among more rows; fall back to 2 when
  // that leaves fewer than two workgroups per CU.  Windowed or block masks
  // always use 2: their key range per workgroup is the window plus the
  // workgroup's rows, so smaller workgroups visit fewer partly-masked tiles.
  const bool banded = m.hi < kInf || m.blk > 0;
  for (int waves : {4, 2}) {
    if (waves == 4 && banded) continue;
    geo.waves = waves;
    geo.rows = 32 * waves;
    const int64_t nblk = (s0 + geo.rows - 1) / geo.rows;
    geo.n_pairs = (int)((nblk + 1) / 2);
    geo.workgroups = batch * heads * geo.residues * geo.n_pairs;
    if (geo.workgroups >= 2 * kCUs) break;
  }
  return geo;
}

// The forward's core and geometry.  Head dim 64: the paired core, or for a
// window or block mask, causal rows with a prefix, and causal softmax on the
// grids named below, the one-block core at four wavefronts per SIMD (north
// star: local 53.2 -> 42.6 us, sliding window 53.1 -> 42.9, block-diagonal
// 39.0 -> 30.5, dilated 61.6 -> 57.5; cold-cache 12-20 % less).  Head dim
// 128: the one-block core (two wavefronts per SIMD), except for sigmoid and
// ReLU on full rows (no causal pairing, window or block) of 2048 keys or more
// without a score modifier and with two 4-wavefront workgroups per CU, where
// the paired core's pipelined run and its K/V tiles shared by two row blocks
// measured faster (B4 H16 D128, sigmoid / ReLU: 141.8 / 122.9 us against
// 155.9 / 129.0 at S2048, 504 / 447 against 533 / 465 at S4096; at S1024 the
// one-block core wins, 45.5 against 61.1 us for sigmoid).  Softmax on such
// rows runs the one-block core: the paired softmax kernel at head_dim 128
// spills (17 VGPRs at one wavefront per SIMD), and the one-block core
// measured 288.8 against 294.7 us (B4 H16 S4096, temperature).
Geometry forward_geometry(const chia_attn_args* a, const MaskSpec& m, const ScorePath& sp) {
  Geometry geo = paired_geometry(m, a->batch, a->heads);
  const bool banded = m.hi < kInf || m.blk > 0;
  const int32_t s0 = residue_geom(m, 0).S;
  // Causal rows with a prefix every query sees: a row block's work is the
  // prefix or its causal band, whichever is longer, which zigzag pairs do not
  // balance.  At head dim 64 such rows run the one-block core, one block per
  // workgroup, the blocks with the most keys launched first (prefix-LM 1024,
  // B4 H16 D64: 173.3 -> 164.0 us at S4096, 62.6 -> 56.9 us at S2048; the same
  // order on the paired core, 166.0 / 62.3 us).
  const bool prefix_causal = geo.zigzag && m.prefix > 0;
  // Plain causal softmax at head dim 64 runs the one-block core too, blocks
  // longest-first, on the grids where it measured faster than the zigzag pairs
  // (temperature + ALiBi + softcap, us, one process):
  //   * pairs on 2-wavefront workgroups (too few rows for two 4-wavefront ones
  //     per CU) and at least two one-block workgroups per CU: B4 H16 S1024
  //     97.6 -> 79.6, B2 H16 S2048 164.2 -> 136.0, B1 H16 S4096 302.5 -> 252.8;
  //     with fewer, slower (B1 H8 S2048, 128 workgroups: 122.7 -> 131.8);
  //   * at least 64 (batch, head, residue) slices of at most 4096 rows:
  //     B4 H16 S2048 169.8 -> 166.7, B4 H16 S4096 534.0 -> 517.5, B8 H32 S1024
  //     195.5 -> 172.1; with 32 slices slower (B2 H16 S4096 294.5 -> 312.9),
  //     and at 8192 rows slower or even (B1 H16 524.1 -> 578.2, B4 H16
  //     2023 -> 2032).
  // Only where the longest-first order applies (it needs a multiple of 8
  // slices and no packed sequences): in natural order the blocks' unequal work
  // is not balanced.  Full rows keep the paired core (north star, temperature
  // 281.3 -> 302.6 us).
  bool causal_q1 = false;
  if (a->head_dim == 64 && geo.zigzag && !prefix_causal && !banded && a->norm == CHIA_ATTN_NORM_SOFTMAX &&
      s0 <= 4096 && !a->cu_seqlens) {
    const int64_t slices = a->batch * a->heads * geo.residues;
    const int64_t q1_wg = slices * ((s0 + 127) / 128);
    causal_q1 = slices % 8 == 0 && (slices >= 64 || (geo.waves == 2 && q1_wg >= 2 * kCUs));
  }
  if (a->head_dim == 64 && !banded && !prefix_causal && !causal_q1) return geo;
  if (a->head_dim == 128 && a->norm != CHIA_ATTN_NORM_SOFTMAX && !geo.zigzag && !banded && s0 >= 2048 && !sp.alibi &&
      !sp.softcap && geo.waves == 4)
    return geo;
  geo.q1 = true;
  geo.waves = 4;
  geo.rows = 128;
  if (a->head_dim == 64 && (prefix_causal || causal_q1)) {
    geo.zigzag = 0;
    geo.rank = true;
  }
  const int64_t nblk = (s0 + geo.rows - 1) / geo.rows;
  geo.n_pairs = (int)(geo.zigzag ? (nblk + 1) / 2 : nblk);
  geo.workgroups = a->batch * a->heads * geo.residues * geo.n_pairs;
  // Head dim 128, zigzag pairs on fewer than two workgroups per CU: one group
  // per workgroup would leave one wavefront per SIMD, so two groups split
  // each pair's steps (every SIMD then holds two wavefronts).
  if (a->head_dim == 128 && geo.zigzag && geo.workgroups < 2 * kCUs) geo.groups = 2;
  return geo;
}

}  // namespace
}  // namespace chia

using namespace chia;

extern "C" int chia_attn_abi_version(void) { return CHIA_ATTN_ABI_VERSION; }

extern "C" const char* chia_attn_status_string(int status) {
  switch (status) {
    case CHIA_ATTN_OK: return "ok";
    case CHIA_ATTN_ERR_NULL: return "null argument, tensor or required per-head pointer";
    case CHIA_ATTN_ERR_SHAPE:
      return "batch, heads and seqlen must be >= 1 (seqlen < 2^28); K/V seq strides in [0, 2^25 / dilation); "
             "kv_heads >= 0 and dividing heads";
    case CHIA_ATTN_ERR_HEAD_DIM: return "head_dim must be 64 or 128";
    case CHIA_ATTN_ERR_MASK: return "window, block and prefix must be >= 0, dilation >= 1, and prefix is not combinable with dilation > 1";
    case CHIA_ATTN_ERR_SCALE: return "scale must be finite and > 0; softcap finite and >= 0; bias, post_scale finite";
    case CHIA_ATTN_ERR_NORM: return "unknown normaliser";
    case CHIA_ATTN_ERR_ALIGN: return "tensors must be 16-byte aligned with batch/head/seq strides multiple of 8 elements";
    case CHIA_ATTN_ERR_STRUCT: return "struct_size mismatch or reserved fields not zero";
    case CHIA_ATTN_ERR_WORKSPACE: return "backward workspace NULL or smaller than chia_attn_bwd_workspace_size";
    case CHIA_ATTN_ERR_SCRATCH:
      return "chia_attn_bwd_noalloc: the row statistics (chia_attn_bwd_workspace_size bytes) exceed the static "
             "scratch of CHIA_ATTN_NOALLOC_SCRATCH_BYTES";
    default: break;
  }
  if (status > 0) return hipGetErrorString((hipError_t)status);
  return "unknown status";
}

namespace {
int launch_fwd(const chia_attn_args* a, float* lse, void* stream) {
  const int st = validate(a, true);
  if (st != CHIA_ATTN_OK) return st;
  if ((uintptr_t)lse & 3u) return CHIA_ATTN_ERR_ALIGN;

  FwdParams p;
  std::memset(&p, 0, sizeof(p));
  p.q = (const uint16_t*)a->q;
  p.k = (const uint16_t*)a->k;
  p.v = (const uint16_t*)a->v;
  p.o = (uint16_t*)a->o;
  p.q_sb = batch_stride(a, a->q_stride); p.q_sh = a->q_stride[1]; p.q_ss = a->q_stride[2];
  p.k_sb = batch_stride(a, a->k_stride); p.k_sh = a->k_stride[1]; p.k_ss = a->k_stride[2];
  p.v_sb = batch_stride(a, a->v_stride); p.v_sh = a->v_stride[1]; p.v_ss = a->v_stride[2];
  p.o_sb = batch_stride(a, a->o_stride); p.o_sh = a->o_stride[1]; p.o_ss = a->o_stride[2];
  p.head_scale = a->head_scale;
  p.alibi_slopes = a->alibi_slopes;
  p.mask = spec_of(a);
  p.B = (int32_t)a->batch;
  p.H = (int32_t)a->heads;
  p.cu_seqlens = a->cu_seqlens;
  p.seq_order = a->cu_seqlens ? a->seq_order : nullptr;
  // lse: [B, H, S], or [T, H] for packed sequences
  p.lse_sb = a->cu_seqlens ? 0 : a->heads * a->seqlen;
  p.lse_sh = a->cu_seqlens ? 1 : a->seqlen;
  p.lse_ss = a->cu_seqlens ? a->heads : 1;
  const ScorePath sp = score_path_of(a);
  const Geometry geo = forward_geometry(a, p.mask, sp);
  p.residues = geo.residues;
  p.n_pairs = geo.n_pairs;
  p.zigzag = geo.zigzag;
  const int waves = geo.waves;
  if (geo.workgroups >= ((int64_t)1 << 31)) return CHIA_ATTN_ERR_SHAPE;
  p.n_wg = (int32_t)geo.workgroups;
  const int64_t slices = a->batch * a->heads * p.residues;
  if (geo.rank && !a->cu_seqlens && slices % 8 == 0) p.rank_hx = (int32_t)(slices / 8);
  p.div_hx = make_udiv(p.rank_hx > 0 ? p.rank_hx : 1);
  p.div_pairs = make_udiv(p.n_pairs);
  p.div_res = make_udiv(p.residues);
  p.div_h = make_udiv(p.H);
  p.div_group = make_udiv(a->kv_heads > 0 ? (int32_t)(a->heads / a->kv_heads) : 1);
  p.scale = a->scale;
  p.softcap = a->softcap;
  p.bias = a->bias;
  p.post_scale = a->post_scale;
  p.lse = a->norm == CHIA_ATTN_NORM_SOFTMAX ? lse : nullptr;

  // Softcap softmax on the one-block core: weights against a fixed reference
  // when cap log2 e <= 78 (cap <= 54), which keeps every weight normal
  // (attn_fwd_q1_kernel.h); north star 208.7 -> 200.6 us, headline 66.7 ->
  // 62.7 us against the running max.
  const bool cap_fixed = sp.softcap && a->norm == CHIA_ATTN_NORM_SOFTMAX && a->softcap * kLog2e <= 78.0f;
  KernelFn fn = a->head_dim == 64 ? (geo.q1 ? select_q1_kernel_d64((int)a->norm, sp.alibi, sp.softcap, cap_fixed)
                                            : select_kernel_d64(waves, (int)a->norm, sp.alibi, sp.softcap))
               : geo.q1            ? (geo.groups == 2 ? select_q1_split_kernel_d128((int)a->norm, sp.alibi, sp.softcap, cap_fixed)
                                                  : select_q1_kernel_d128((int)a->norm, sp.alibi, sp.softcap, cap_fixed))
                                   : select_kernel_d128((int)a->norm);
  if (fn == nullptr) return CHIA_ATTN_ERR_NORM;  // no instantiation for this core and normaliser
  void* kargs[] = {&p};
  hipError_t err = hipLaunchKernel(reinterpret_cast<const void*>(fn), dim3((unsigned)p.n_wg),
                                   dim3(64 * waves * geo.groups), kargs, 0, (hipStream_t)stream);
  if (err != hipSuccess) return (int)err;
  err = hipGetLastError();
  return err == hipSuccess ? CHIA_ATTN_OK : (int)err;
}
}  // namespace

extern "C" int chia_attn_fwd(const chia_attn_args* a, void* stream) { return launch_fwd(a, nullptr, stream); }

extern "C" int chia_attn_fwd_lse(const chia_attn_args* a, float* lse, void* stream) {
  if (lse == nullptr && a != nullptr && a->norm == CHIA_ATTN_NORM_SOFTMAX) return CHIA_ATTN_ERR_NULL;
  return launch_fwd(a, lse, stream);
}

namespace {
constexpr int kBwdMaxGroup = 256;  // query heads per K/V head the dK/dV kernel stages
constexpr int kBwdBlock = 128;     // rows (dQ) or keys (dK/dV) per workgroup

// Rows of the stats workspace per (b, h, residue): residue 0's length padded
// to the 64-row tiles the dK/dV kernel reads whole.
int64_t stats_rows(const MaskSpec& m) { return ((int64_t)residue_geom(m, 0).S + 63) / 64 * 64; }

int64_t bwd_workspace(const chia_attn_args* a) {
  if (a->norm != CHIA_ATTN_NORM_SOFTMAX) return 0;
  const MaskSpec m = spec_of(a);
  return 2 * a->batch * a->heads * (int64_t)num_residues(m) * stats_rows(m) * (int64_t)sizeof(float);
}

hipError_t launch(BwdKernelFn fn, int64_t grid, const BwdParams& p, hipStream_t stream) {
  if (grid <= 0) return hipSuccess;
  BwdParams q = p;
  q.n_wg = (int32_t)grid;
  void* kargs[] = {&q};
  const hipError_t err = hipLaunchKernel(reinterpret_cast<const void*>(fn), dim3((unsigned)grid), dim3(256), kargs, 0, stream);
  return err != hipSuccess ? err : hipGetLastError();
}
}  // namespace

extern "C" int64_t chia_attn_bwd_workspace_size(const chia_attn_args* a) {
  const int st = validate(a, false);
  return st != CHIA_ATTN_OK ? st : bwd_workspace(a);
}

// ---- allocation-free backward: the row statistics in a static device array -----
// `scratch` is a file-scope device array: each GPU the library runs on holds its
// own copy (allocated with the code object, held until the process ends).  In
// host code its name is only a stand-in for the symbol; the device address is
// taken once per device with hipGetSymbolAddress, with that device current, and
// only that address is ever handed to a kernel.
static __device__ __align__(256) char scratch[CHIA_ATTN_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;

// The current device's address of `scratch` (hipGetSymbolAddress on the first
// call on each device).  Returns a chia_attn_status / hipError_t code.
int scratch_address(void** out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess) return (int)err;
  if (dev < 0 || dev >= kMaxDevices) return (int)hipErrorInvalidDevice;
  void* ptr = g_scratch[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    ptr = g_scratch[dev].load(std::memory_order_relaxed);
    if (ptr == nullptr) {
      err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      if (err != hipSuccess) return (int)err;
      if (ptr == nullptr) return (int)hipErrorInvalidSymbol;
      g_scratch[dev].store(ptr, std::memory_order_release);
    }
  }
  *out = ptr;
  return CHIA_ATTN_OK;
}

int launch_bwd(const chia_attn_bwd_args* ba, void* stream, bool noalloc);
}  // namespace

extern "C" int chia_attn_bwd(const chia_attn_bwd_args* ba, void* stream) { return launch_bwd(ba, stream, false); }

extern "C" int chia_attn_bwd_noalloc(const chia_attn_bwd_args* ba, void* stream) {
  return launch_bwd(ba, stream, true);
}

namespace {
// chia_attn_bwd; with `noalloc` the row statistics go to the current device's
// `scratch` instead of the caller's workspace (whose fields are then ignored).
int launch_bwd(const chia_attn_bwd_args* ba, void* stream, bool noalloc) {
  if (!ba) return CHIA_ATTN_ERR_NULL;
  if (ba->struct_size != sizeof(chia_attn_bwd_args) || ba->reserved0 != 0) return CHIA_ATTN_ERR_STRUCT;
  for (int i = 0; i < 8; ++i)
    if (ba->reserved[i] != 0) return CHIA_ATTN_ERR_STRUCT;
  const chia_attn_args* a = ba->fwd;
  const int st = validate(a, true);
  if (st != CHIA_ATTN_OK) return st;
  if (!ba->dout || !ba->dq || !ba->dk || !ba->dv) return CHIA_ATTN_ERR_NULL;
  if (!aligned16(ba->dout) || !aligned16(ba->dq) || !aligned16(ba->dk) || !aligned16(ba->dv)) return CHIA_ATTN_ERR_ALIGN;
  if (!stride_ok(ba->dout_stride) || !stride_ok(ba->dq_stride) || !stride_ok(ba->dk_stride) || !stride_ok(ba->dv_stride))
    return CHIA_ATTN_ERR_ALIGN;
  // Q and dO tiles are streamed like K and V: 32-bit row offsets within a tile
  for (const int64_t* s : {a->q_stride, ba->dout_stride})
    if (s[2] < 0 || s[2] * a->dilation >= kMaxKvRowStride) return CHIA_ATTN_ERR_SHAPE;
  const bool softmax = a->norm == CHIA_ATTN_NORM_SOFTMAX;
  void* stats = nullptr;
  if (softmax) {
    if (!ba->lse) return CHIA_ATTN_ERR_NULL;
    if ((uintptr_t)ba->lse & 3u) return CHIA_ATTN_ERR_ALIGN;
    if (noalloc) {
      if (bwd_workspace(a) > (int64_t)CHIA_ATTN_NOALLOC_SCRATCH_BYTES) return CHIA_ATTN_ERR_SCRATCH;
    } else {
      if (!ba->workspace || ba->workspace_bytes < bwd_workspace(a) || ((uintptr_t)ba->workspace & 15u))
        return CHIA_ATTN_ERR_WORKSPACE;
      stats = ba->workspace;
    }
  }
  const int64_t hkv = a->kv_heads > 0 ? a->kv_heads : a->heads;
  const int64_t G = a->heads / hkv;
  if (G > kBwdMaxGroup) return CHIA_ATTN_ERR_SHAPE;
  if (softmax && noalloc) {
    const int st_s = scratch_address(&stats);
    if (st_s != CHIA_ATTN_OK) return st_s;
  }

  BwdParams p;
  std::memset(&p, 0, sizeof(p));
  p.q = (const uint16_t*)a->q;
  p.k = (const uint16_t*)a->k;
  p.v = (const uint16_t*)a->v;
  p.o = (const uint16_t*)a->o;
  p.dout = (const uint16_t*)ba->dout;
  p.dq = (uint16_t*)ba->dq;
  p.dk = (uint16_t*)ba->dk;
  p.dv = (uint16_t*)ba->dv;
  p.q_sb = batch_stride(a, a->q_stride); p.q_sh = a->q_stride[1]; p.q_ss = a->q_stride[2];
  p.k_sb = batch_stride(a, a->k_stride); p.k_sh = a->k_stride[1]; p.k_ss = a->k_stride[2];
  p.v_sb = batch_stride(a, a->v_stride); p.v_sh = a->v_stride[1]; p.v_ss = a->v_stride[2];
  p.o_sb = batch_stride(a, a->o_stride); p.o_sh = a->o_stride[1]; p.o_ss = a->o_stride[2];
  p.do_sb = batch_stride(a, ba->dout_stride); p.do_sh = ba->dout_stride[1]; p.do_ss = ba->dout_stride[2];
  p.dq_sb = batch_stride(a, ba->dq_stride); p.dq_sh = ba->dq_stride[1]; p.dq_ss = ba->dq_stride[2];
  p.dk_sb = batch_stride(a, ba->dk_stride); p.dk_sh = ba->dk_stride[1]; p.dk_ss = ba->dk_stride[2];
  p.dv_sb = batch_stride(a, ba->dv_stride); p.dv_sh = ba->dv_stride[1]; p.dv_ss = ba->dv_stride[2];
  p.cu_seqlens = a->cu_seqlens;
  p.seq_order = a->cu_seqlens ? a->seq_order : nullptr;
  p.lse = softmax ? ba->lse : nullptr;
  p.lse_sb = a->cu_seqlens ? 0 : a->heads * a->seqlen;
  p.lse_sh = a->cu_seqlens ? 1 : a->seqlen;
  p.lse_ss = a->cu_seqlens ? a->heads : 1;
  p.stats = (float*)stats;
  p.head_scale = a->head_scale;
  p.alibi_slopes = a->alibi_slopes;
  p.mask = spec_of(a);
  p.B = (int32_t)a->batch;
  p.H = (int32_t)a->heads;
  p.G = (int32_t)G;
  p.residues = num_residues(p.mask);
  p.SR = (int32_t)stats_rows(p.mask);
  p.n_blk = (residue_geom(p.mask, 0).S + kBwdBlock - 1) / kBwdBlock;
  p.div_blk = make_udiv(p.n_blk);
  p.div_res = make_udiv(p.residues);
  p.div_h = make_udiv(p.H);
  p.div_g = make_udiv(p.G);
  p.div_hk = make_udiv((int32_t)hkv);
  p.div_dil = make_udiv(p.mask.dil);
  p.scale = a->scale;
  p.softcap = a->softcap;
  p.bias = a->bias;
  p.post_scale = a->post_scale;

  const int64_t g_dq = a->batch * a->heads * p.residues * (int64_t)p.n_blk;
  const int64_t g_dkdv = a->batch * hkv * p.residues * (int64_t)p.n_blk;
  if (g_dq >= ((int64_t)1 << 31)) return CHIA_ATTN_ERR_SHAPE;

  const bool alibi = a->alibi_slopes != nullptr, softcap = a->softcap > 0.f;
  const BwdKernels ks = a->head_dim == 64 ? select_bwd_kernels_d64((int)a->norm, alibi, softcap)
                                          : select_bwd_kernels_d128((int)a->norm, alibi, softcap);
  const hipStream_t s = (hipStream_t)stream;
  hipError_t err = hipSuccess;
  // dQ first: with softmax it also writes the row statistics dK/dV reads.
  // Causal rows: each kernel launches its blocks with the most work first
  // (rank_order): the last query blocks (dQ), the first key blocks (dK/dV).
  auto rank_for = [&](int64_t slices) {
    const bool on = zigzag_of(p.mask) && !a->cu_seqlens && slices % 8 == 0;
    p.rank_hx = on ? (int32_t)(slices / 8) : 0;
    p.div_hx = make_udiv(on ? p.rank_hx : 1);
  };
  rank_for(a->batch * a->heads * p.residues);
  err = launch(ks.dq, g_dq, p, s);
  rank_for(a->batch * hkv * p.residues);
  // a group whose query heads differ in scale takes c1 per score
  const BwdKernelFn dkdv = G > 1 && a->head_scale ? ks.dkdv_head_c1 : ks.dkdv;
  if (err == hipSuccess) err = launch(dkdv, g_dkdv, p, s);
  return err == hipSuccess ? CHIA_ATTN_OK : (int)err;
}
}  // namespace

extern "C" int chia_attn_fwd_fp8(const chia_attn_fp8_args* fa, void* stream) {
  if (!fa) return CHIA_ATTN_ERR_NULL;
  if (fa->struct_size != sizeof(chia_attn_fp8_args) || fa->format > CHIA_ATTN_FP8_E5M2) return CHIA_ATTN_ERR_STRUCT;
  for (int i = 0; i < 5; ++i)
    if (fa->reserved[i] != 0) return CHIA_ATTN_ERR_STRUCT;
  const chia_attn_args* a = fa->attn;
  const int st = validate(a, true);
  if (st != CHIA_ATTN_OK) return st;
  for (float d : {fa->q_descale, fa->k_descale, fa->v_descale})
    if (!(d > 0.f) || !std::isfinite(d)) return CHIA_ATTN_ERR_SCALE;
  // fp8 rows are D bytes: the 16-byte DMA chunks need byte strides that are multiples of 16
  for (const int64_t* s : {a->q_stride, a->k_stride, a->v_stride})
    if (s[0] % 16 || s[1] % 16 || s[2] % 16) return CHIA_ATTN_ERR_ALIGN;
  if (a->q_stride[2] * a->dilation >= kMaxKvRowStride) return CHIA_ATTN_ERR_SHAPE;

  Fp8Params p;
  std::memset(&p, 0, sizeof(p));
  p.q = (const uint8_t*)a->q;
  p.k = (const uint8_t*)a->k;
  p.v = (const uint8_t*)a->v;
  p.o = (uint16_t*)a->o;
  p.q_sb = batch_stride(a, a->q_stride); p.q_sh = a->q_stride[1]; p.q_ss = a->q_stride[2];
  p.k_sb = batch_stride(a, a->k_stride); p.k_sh = a->k_stride[1]; p.k_ss = a->k_stride[2];
  p.v_sb = batch_stride(a, a->v_stride); p.v_sh = a->v_stride[1]; p.v_ss = a->v_stride[2];
  p.o_sb = batch_stride(a, a->o_stride); p.o_sh = a->o_stride[1]; p.o_ss = a->o_stride[2];
  p.cu_seqlens = a->cu_seqlens;
  p.seq_order = a->cu_seqlens ? a->seq_order : nullptr;
  p.head_scale = a->head_scale;
  p.alibi_slopes = a->alibi_slopes;
  p.mask = spec_of(a);
  p.B = (int32_t)a->batch;
  p.H = (int32_t)a->heads;
  p.residues = num_residues(p.mask);
  p.n_blk = (residue_geom(p.mask, 0).S + 127) / 128;
  const int64_t bhr = a->batch * a->heads * p.residues;
  const int64_t n_wg = bhr * (int64_t)p.n_blk;
  // Causal rows without a window: a block's work grows with its index, and the
  // launch walks the longest blocks of every slice first (per XCD).
  if (zigzag_of(p.mask) && !a->cu_seqlens && bhr % 8 == 0) p.rank_hx = (int32_t)(bhr / 8);
  p.div_hx = make_udiv(p.rank_hx > 0 ? p.rank_hx : 1);
  if (n_wg >= ((int64_t)1 << 31)) return CHIA_ATTN_ERR_SHAPE;
  p.n_wg = (int32_t)n_wg;
  p.div_blk = make_udiv(p.n_blk);
  p.div_res = make_udiv(p.residues);
  p.div_h = make_udiv(p.H);
  p.div_group = make_udiv(a->kv_heads > 0 ? (int32_t)(a->heads / a->kv_heads) : 1);
  p.qk_scale = a->scale * fa->q_descale * fa->k_descale;
  p.v_descale = fa->v_descale;
  p.softcap = a->softcap;
  p.bias = a->bias;
  p.post_scale = a->post_scale;
  const Fp8KernelFn fn = select_fp8_kernel((int)a->head_dim, (int)fa->format, (int)a->norm, a->alibi_slopes != nullptr,
                                           a->softcap > 0.f);
  if (!fn) return CHIA_ATTN_ERR_NORM;
  void* kargs[] = {&p};
  hipError_t err = hipLaunchKernel(reinterpret_cast<const void*>(fn), dim3((unsigned)p.n_wg), dim3(256), kargs, 0,
                                   (hipStream_t)stream);
  if (err != hipSuccess) return (int)err;
  err = hipGetLastError();
  return err == hipSuccess ? CHIA_ATTN_OK : (int)err;
}

extern "C" int chia_attn_plan(const chia_attn_args* a, chia_attn_plan_info* out) {
  const int st = validate(a, false);
  if (st != CHIA_ATTN_OK) return st;
  if (!out) return CHIA_ATTN_ERR_NULL;
  std::memset(out, 0, sizeof(*out));
  const MaskSpec spec = spec_of(a);
  const Geometry geo = forward_geometry(a, spec, score_path_of(a));
  const int bn = kBN;
  const int64_t bhn = a->batch * a->heads;
  // The paired core computes two row blocks per KV tile in 32 x 64 sub-tiles;
  // the one-block core one row block per KV tile, in 32-key steps.
  out->block_m = geo.q1 ? geo.rows : 2 * geo.rows;  // rows per workgroup step
  out->block_n = geo.q1 ? bn / 2 : bn;                // keys per computed step
  out->wave_m = 32;  // visited-tile unit: 32 rows x block_n keys
  out->waves = geo.waves;
  out->residues = geo.residues;
  out->workgroups = geo.workgroups;
  int64_t tiles_total = 0, tiles_visited = 0, wave_tiles = 0, wave_partial = 0, pairs = 0;
  for (int r = 0; r < geo.residues; ++r) {
    const MaskGeom g = residue_geom(spec, r);
    if (g.S <= 0) continue;
    const int64_t nkt = (g.S + bn - 1) / bn;
    const int nblk = (g.S + geo.rows - 1) / geo.rows;
    if (geo.q1) {
      // every row block once (by its workgroup), its own key range, 32-key
      // steps a wavefront skips when none of its rows sees them
      tiles_total += (int64_t)nblk * 2 * nkt;
      for (int blk = 0; blk < nblk; ++blk) {
        const TileRange tr = tile_range(g, blk * geo.rows, imin32(blk * geo.rows + geo.rows - 1, g.S - 1), bn);
        const int n = tr.n_pre + tr.n2;
        tiles_visited += 2 * n;
        for (int it = 0; it < n; ++it)
          for (int w = 0; w < geo.waves; ++w) {
            const int32_t r0 = blk * geo.rows + 32 * w;
            if (r0 >= g.S) continue;
            for (int kb = 0; kb < 2; ++kb) {
              const int32_t c = tile_at(tr, it) * bn + 32 * kb;
              const int cls = classify_tile(g, r0, imin32(r0 + 31, g.S - 1), c, c + 31);
              if (cls != TILE_EMPTY) ++wave_tiles;
              if (cls == TILE_PARTIAL) ++wave_partial;
            }
          }
      }
    } else {
      tiles_total += (int64_t)((nblk + 1) / 2) * nkt;
      for (int pr = 0; pr < geo.n_pairs; ++pr) {
        int b0, b1;
        if (geo.zigzag) {
          b0 = pr;
          b1 = nblk - 1 - pr;
          if (b1 < b0) continue;
          if (b1 == b0) b1 = -1;
        } else {
          b0 = 2 * pr;
          b1 = 2 * pr + 1;
          if (b0 >= nblk) continue;
          if (b1 >= nblk) b1 = -1;
        }
        const int32_t hull_hi = imin32((b1 >= 0 ? b1 : b0) * geo.rows + geo.rows - 1, g.S - 1);
        const TileRange tr = tile_range(g, b0 * geo.rows, hull_hi, bn);
        const int n = tr.n_pre + tr.n2;
        tiles_visited += n;
        for (int it = 0; it < n; ++it) {
          const int32_t jt0 = tile_at(tr, it) * bn;
          for (int blk : {b0, b1}) {
            if (blk < 0) continue;
            for (int w = 0; w < geo.waves; ++w) {
              const int32_t r0 = blk * geo.rows + 32 * w;
              if (r0 >= g.S) continue;
              const int cls = classify_tile(g, r0, imin32(r0 + 31, g.S - 1), jt0, jt0 + bn - 1);
              if (cls != TILE_EMPTY) ++wave_tiles;
              if (cls == TILE_PARTIAL) ++wave_partial;
            }
          }
        }
      }
    }
    for (int32_t i = 0; i < g.S; ++i) {
      const int32_t lo = imax32(key_lo(g, i), g.prefix), hi = key_hi(g, i);
      pairs += g.prefix + (hi >= lo ? hi - lo + 1 : 0);
    }
  }
  out->tiles_total = tiles_total * bhn;
  out->tiles_visited = tiles_visited * bhn;
  out->wave_tiles_visited = wave_tiles * bhn;
  out->wave_tiles_partial = wave_partial * bhn;
  out->pairs_visible = pairs * bhn;
  return CHIA_ATTN_OK;
}

extern "C" int chia_attn_tile_map(const chia_attn_args* a, int32_t residue, int32_t rows_per_block, int32_t* n_qb,
                                  int32_t* n_kt, int8_t* out, int64_t out_len) {
  const int st = validate(a, false);
  if (st != CHIA_ATTN_OK) return st;
  if (!n_qb || !n_kt) return CHIA_ATTN_ERR_NULL;
  const MaskSpec spec = spec_of(a);
  if (residue < 0 || residue >= num_residues(spec) || rows_per_block < 1) return CHIA_ATTN_ERR_MASK;
  const MaskGeom g = residue_geom(spec, residue);
  const int bn = kBN;
  *n_qb = (g.S + rows_per_block - 1) / rows_per_block;
  *n_kt = (g.S + bn - 1) / bn;
  if (!out) return CHIA_ATTN_OK;
  if (out_len < (int64_t)(*n_qb) * (*n_kt)) return CHIA_ATTN_ERR_SHAPE;
  for (int32_t qb = 0; qb < *n_qb; ++qb) {
    const int32_t a0 = qb * rows_per_block, a1 = imin32(a0 + rows_per_block - 1, g.S - 1);
    for (int32_t kt = 0; kt < *n_kt; ++kt)
      out[(int64_t)qb * (*n_kt) + kt] = (int8_t)classify_tile(g, a0, a1, kt * bn, kt * bn + bn - 1);
  }
  return CHIA_ATTN_OK;
}

extern "C" int chia_attn_query_intervals(const chia_attn_args* a, int32_t residue, int32_t* jlo, int32_t* jhi,
                                         int32_t* prefix_len, int64_t len) {
  const int st = validate(a, false);
  if (st != CHIA_ATTN_OK) return st;
  if (!jlo || !jhi || !prefix_len) return CHIA_ATTN_ERR_NULL;
  const MaskSpec spec = spec_of(a);
  if (residue < 0 || residue >= num_residues(spec)) return CHIA_ATTN_ERR_MASK;
  const MaskGeom g = residue_geom(spec, residue);
  if (len < g.S) return CHIA_ATTN_ERR_SHAPE;
  for (int32_t i = 0; i < g.S; ++i) {
    jlo[i] = key_lo(g, i);
    jhi[i] = key_hi(g, i);
  }
  *prefix_len = g.prefix;
  return CHIA_ATTN_OK;
}
