// attn_api.hip -- the C ABI (include/chia_attn.h): argument validation, the
// launch of the gfx950 core, and the host-only planning entry points.
//
// Reference boundary replaced: launch_kernel(q, k, v) -> o of
// kernels_gemini31propre_0018/<op>_BEST.py (e.g. bias_sliding_window_BEST.py:87-108).
// Unlike the reference (callee allocates o, shapes baked into each kernel),
// the caller passes o and every variant parameter explicitly.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>

#include "attn_fwd_kernel.h"
#include "chia_attn.h"

namespace chia {

using KernelFn = void (*)(FwdParams);
KernelFn select_kernel_d64(int norm, bool alibi, bool softcap);
KernelFn select_kernel_d128(int norm, bool alibi, bool softcap);

namespace {

constexpr int64_t kMaxSeq = (int64_t)1 << 28;

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
  for (int i = 0; i < 8; ++i)
    if (a->reserved[i] != 0) return CHIA_ATTN_ERR_STRUCT;
  if (need_tensors) {
    if (!aligned16(a->q) || !aligned16(a->k) || !aligned16(a->v) || !aligned16(a->o)) return CHIA_ATTN_ERR_ALIGN;
    if (!stride_ok(a->q_stride) || !stride_ok(a->k_stride) || !stride_ok(a->v_stride) || !stride_ok(a->o_stride))
      return CHIA_ATTN_ERR_ALIGN;
    if (((uintptr_t)a->head_scale & 3u) || ((uintptr_t)a->alibi_slopes & 3u)) return CHIA_ATTN_ERR_ALIGN;
  }
  return CHIA_ATTN_OK;
}

MaskSpec spec_of(const chia_attn_args* a) {
  return make_mask_spec((int32_t)a->seqlen, a->causal ? 1 : 0, a->window, a->dilation, a->block, a->prefix);
}

int block_m_of(int64_t head_dim) {
  return kWaves * 32 * (head_dim == 64 ? TileCfg<64>::QB : TileCfg<128>::QB);
}

int wave_m_of(int64_t head_dim) { return 32 * (head_dim == 64 ? TileCfg<64>::QB : TileCfg<128>::QB); }

}  // namespace
}  // namespace chia

using namespace chia;

extern "C" int chia_attn_abi_version(void) { return CHIA_ATTN_ABI_VERSION; }

extern "C" const char* chia_attn_status_string(int status) {
  switch (status) {
    case CHIA_ATTN_OK: return "ok";
    case CHIA_ATTN_ERR_NULL: return "null argument, tensor or required per-head pointer";
    case CHIA_ATTN_ERR_SHAPE: return "batch, heads and seqlen must be >= 1 (seqlen < 2^28)";
    case CHIA_ATTN_ERR_HEAD_DIM: return "head_dim must be 64 or 128";
    case CHIA_ATTN_ERR_MASK: return "window, block and prefix must be >= 0, dilation >= 1, and prefix is not combinable with dilation > 1";
    case CHIA_ATTN_ERR_SCALE: return "scale must be finite and > 0; softcap finite and >= 0; bias, post_scale finite";
    case CHIA_ATTN_ERR_NORM: return "unknown normaliser";
    case CHIA_ATTN_ERR_ALIGN: return "tensors must be 16-byte aligned with batch/head/seq strides multiple of 8 elements";
    case CHIA_ATTN_ERR_STRUCT: return "struct_size mismatch or reserved fields not zero";
    default: break;
  }
  if (status > 0) return hipGetErrorString((hipError_t)status);
  return "unknown status";
}

extern "C" int chia_attn_fwd(const chia_attn_args* a, void* stream) {
  const int st = validate(a, true);
  if (st != CHIA_ATTN_OK) return st;

  FwdParams p;
  std::memset(&p, 0, sizeof(p));
  p.q = (const uint16_t*)a->q;
  p.k = (const uint16_t*)a->k;
  p.v = (const uint16_t*)a->v;
  p.o = (uint16_t*)a->o;
  p.q_sb = a->q_stride[0]; p.q_sh = a->q_stride[1]; p.q_ss = a->q_stride[2];
  p.k_sb = a->k_stride[0]; p.k_sh = a->k_stride[1]; p.k_ss = a->k_stride[2];
  p.v_sb = a->v_stride[0]; p.v_sh = a->v_stride[1]; p.v_ss = a->v_stride[2];
  p.o_sb = a->o_stride[0]; p.o_sh = a->o_stride[1]; p.o_ss = a->o_stride[2];
  p.head_scale = a->head_scale;
  p.alibi_slopes = a->alibi_slopes;
  p.mask = spec_of(a);
  p.B = (int32_t)a->batch;
  p.H = (int32_t)a->heads;
  p.residues = num_residues(p.mask);
  const int bm = block_m_of(a->head_dim);
  const int32_t s0 = residue_geom(p.mask, 0).S;  // longest residue class
  p.n_qblk = (s0 + bm - 1) / bm;
  const int64_t n_wg = (int64_t)p.B * p.H * p.residues * p.n_qblk;
  if (n_wg >= ((int64_t)1 << 31)) return CHIA_ATTN_ERR_SHAPE;
  p.n_wg = (int32_t)n_wg;
  p.scale = a->scale;
  p.softcap = a->softcap;
  p.bias = a->bias;
  p.post_scale = a->post_scale;

  const bool alibi = a->alibi_slopes != nullptr;
  const bool softcap = a->softcap > 0.f;
  KernelFn fn = a->head_dim == 64 ? select_kernel_d64((int)a->norm, alibi, softcap)
                                  : select_kernel_d128((int)a->norm, alibi, softcap);
  void* kargs[] = {&p};
  hipError_t err = hipLaunchKernel(reinterpret_cast<const void*>(fn), dim3((unsigned)p.n_wg), dim3(kThreads), kargs,
                                   0, (hipStream_t)stream);
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
  const int bm = block_m_of(a->head_dim), wm = wave_m_of(a->head_dim);
  const int bn = kBN;
  const int nres = num_residues(spec);
  const int32_t s0 = residue_geom(spec, 0).S;
  const int64_t n_qblk = (s0 + bm - 1) / bm;
  const int64_t bhn = a->batch * a->heads;
  out->block_m = bm;
  out->block_n = bn;
  out->wave_m = wm;
  out->waves = kWaves;
  out->residues = nres;
  out->workgroups = bhn * nres * n_qblk;
  int64_t tiles_total = 0, tiles_visited = 0, wave_tiles = 0, wave_partial = 0, pairs = 0;
  for (int r = 0; r < nres; ++r) {
    const MaskGeom g = residue_geom(spec, r);
    if (g.S <= 0) continue;
    const int64_t nkt = (g.S + bn - 1) / bn;
    for (int32_t q0 = 0; q0 < g.S; q0 += bm) {
      const int32_t q1 = imin32(q0 + bm - 1, g.S - 1);
      tiles_total += nkt;
      const TileRange tr = tile_range(g, q0, q1, bn);
      const int n = tr.n_pre + tr.n2;
      tiles_visited += n;
      for (int it = 0; it < n; ++it) {
        const int32_t jt0 = tile_at(tr, it) * bn;
        for (int32_t w0 = q0; w0 <= q1; w0 += wm) {
          const int cls = classify_tile(g, w0, imin32(w0 + wm - 1, g.S - 1), jt0, jt0 + bn - 1);
          if (cls != TILE_EMPTY) ++wave_tiles;
          if (cls == TILE_PARTIAL) ++wave_partial;
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
