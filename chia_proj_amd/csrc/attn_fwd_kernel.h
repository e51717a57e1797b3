// attn_fwd_kernel.h -- the gfx950 forward-attention core behind every variant.
//
// Reference semantics: the eager closures of extra_bench.py:32-62 (score
// s = q k^T * scale, score modifier, mask, normaliser in fp32, p rounded to
// bf16, p @ v) and sigmoid_fix.py:34-40 (sigmoid first, then zero the masked
// entries).  This is an original CDNA4 design, not a port of the reference's
// Triton kernels.
//
// Work decomposition
//   * one workgroup = 4 wavefronts = BM query rows of one (batch, head,
//     dilation residue); each wavefront owns QW = 32*QB query rows;
//   * the KV loop walks only the key tiles (BN = 64 keys) the mask can reach
//     (prefix tiles + the band hull); K and V tiles are staged through LDS,
//     double-buffered, one barrier per tile; each wavefront classifies the tile
//     against its own rows and skips it (EMPTY), runs it unmasked (FULL) or
//     with the per-element predicate (PARTIAL).
//
// Matrix-core formulation (v_mfma_f32_32x32x16_bf16, fp32 accumulate)
//   S^T[key, query] = K Q^T : A = K rows (ds_read_b128), B = Q rows kept in
//     VGPRs.  The 32x32 accumulator gives each lane ONE query column and 16
//     keys, so the softmax row max / row sum are in-lane reductions plus one
//     v_permlane32_swap with the other half-wave.
//   O^T[d, query] += V^T P^T : the S^T accumulator registers, rounded to bf16,
//     are directly the B operand (lane = query, keys {0-3, 8-11} for lanes
//     0-31 and {4-7, 12-15} for lanes 32-63 of each 16-key chunk).  The A
//     operand V^T is read from the ROW-MAJOR V tile with two
//     ds_read_b64_tr_b16: within each 16-lane group, lane i receives element
//     (i % 4) of the 8-byte rows addressed by lanes 4e + i/4, e = 0..3, so
//     pointing lane s at V[k0 + s/4][d0 + 4 (s % 4)] hands lane i the four keys
//     k0..k0+3 of column d0 + i -- exactly the key order of the B operand.
//   LDS rows are padded instead of swizzled so that every fragment address is
//   a per-lane base plus a compile-time offset: K rows are 2D+16 bytes apart
//   (the eight rows of a ds_read_b128 phase land on distinct 16-byte bank
//   groups), V rows 2D+32 bytes apart (the four rows x 32 bytes of one
//   transposed-read group do).
//   The softmax runs per 32-key block in the exp2 domain with a lazily moved
//   reference max: the running max (and the O / l rescale) only changes when
//   a block's max exceeds it by more than kRescaleLog2, so p <= 2^kRescaleLog2.
//   The row sum l accumulates the bf16-rounded weights the PV MFMA consumes
//   (v_dot2c_f32_bf16 against (1, 1): one instruction per two weights).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mask.h"

namespace chia {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

enum Norm : int { NORM_SOFTMAX = 0, NORM_SIGMOID = 1, NORM_RELU = 2 };

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleLog2 = 8.0f;  // lazy-rescale threshold (log2 units)
constexpr int kWaves = 4;
constexpr int kThreads = kWaves * 64;
constexpr int kBN = 64;

struct FwdParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  int64_t q_sb, q_sh, q_ss;  // element strides: batch, head, seq
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  const float* head_scale;    // [H] or nullptr
  const float* alibi_slopes;  // [H] or nullptr
  MaskSpec mask;              // original coordinates
  int32_t B, H;
  int32_t residues;           // dilation classes launched
  int32_t n_qblk;             // query blocks per (b, h, residue)
  int32_t n_wg;
  float scale, softcap, bias, post_scale;
};

// Query rows per wavefront (in units of 32) for each head dim.
template <int D>
struct TileCfg {
  static constexpr int QB = (D == 64) ? 2 : 1;
};

template <bool B>
struct BoolTag {
  static constexpr bool value = B;
};

// LDS row pitches (bytes) of the K and V tiles.
template <int D>
struct Pitch {
  static constexpr int K = 2 * D + 16;
  static constexpr int V = 2 * D + 32;
};

// Hardware dispatches workgroup x to XCD x % 8.  Renumber so each XCD runs a
// contiguous range of logical workgroups (the query blocks of the same heads
// share that XCD's L2).  Bijective for any n.
__device__ __forceinline__ int xcd_remap(int x, int n) {
  constexpr int kXcd = 8;
  const int per = (n + kXcd - 1) / kXcd;
  const int tall = n - (per - 1) * kXcd;
  const int xcd = x % kXcd, local = x / kXcd;
  return xcd < tall ? xcd * per + local : tall * per + (xcd - tall) * (per - 1) + local;
}

// max / sum with the other half-wave (lane ^ 32).
__device__ __forceinline__ float xhalf_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xhalf_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
constexpr bf16x2_t kOnes2 = {(__bf16)1.0f, (__bf16)1.0f};

// Two floats -> packed bf16 pair (one v_cvt_pk_bf16_f32, round to nearest even).
__device__ __forceinline__ bf16x2_t pack2(float a, float b) {
  bf16x2_t r;
  r[0] = (__bf16)a;
  r[1] = (__bf16)b;
  return r;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) { return __builtin_bit_cast(uint32_t, pack2(a, b)); }

template <int D, int QB, int NORM, bool ALIBI, bool SOFTCAP>
__global__ __launch_bounds__(kThreads, 2) void attn_fwd_kernel(const FwdParams p) {
  constexpr int BN = kBN;
  constexpr int QW = 32 * QB;        // query rows per wavefront
  constexpr int BM = kWaves * QW;    // query rows per workgroup
  constexpr int KB = BN / 32;        // 32-key blocks per tile
  constexpr int DK = D / 16;         // k-steps of the QK^T MFMA
  constexpr int DB = D / 32;         // 32-row d blocks of O^T
  constexpr int DQ = D / 8;          // 16-byte chunks per K/V row
  constexpr int NLD = BN * DQ / kThreads;  // 16-byte chunks per thread per tile (each of K, V)
  constexpr int KP = Pitch<D>::K, VP = Pitch<D>::V;
  constexpr int K_BYTES = BN * KP;
  constexpr int STAGE_BYTES = K_BYTES + BN * VP;  // K tile + V tile
  static_assert(NLD >= 1, "tile too small for the workgroup");
  constexpr bool kPlainSoftmax = (NORM == NORM_SOFTMAX) && !ALIBI && !SOFTCAP;
  constexpr bool kRawRelu = (NORM == NORM_RELU) && !ALIBI && !SOFTCAP;

  __shared__ __attribute__((aligned(16))) char lds[2 * STAGE_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane & 31, lh = lane >> 5;

  // ---- workgroup -> (batch, head, residue, query block) --------------------
  const int L = xcd_remap(blockIdx.x, p.n_wg);
  const int bhr = L / p.n_qblk;
  const int qblk = p.n_qblk - 1 - (L % p.n_qblk);  // heaviest (last) rows first
  const int r = bhr % p.residues;
  const int bh = bhr / p.residues;
  const int h = bh % p.H, b = bh / p.H;
  const MaskGeom g = residue_geom(p.mask, r);
  const int q0 = qblk * BM;
  if (q0 >= g.S) return;  // whole workgroup, before any barrier

  const int dil = p.mask.dil;
  const uint16_t* qh = p.q + b * p.q_sb + h * p.q_sh + r * p.q_ss;
  const uint16_t* kh = p.k + b * p.k_sb + h * p.k_sh + r * p.k_ss;
  const uint16_t* vh = p.v + b * p.v_sb + h * p.v_sh + r * p.v_ss;
  uint16_t* oh = p.o + b * p.o_sb + h * p.o_sh + r * p.o_ss;
  const int64_t qrs = p.q_ss * dil, krs = p.k_ss * dil, vrs = p.v_ss * dil, ors = p.o_ss * dil;

  // ---- per-head score constants --------------------------------------------
  const float hs = p.head_scale ? p.head_scale[h] : 1.0f;
  const float slope = ALIBI ? p.alibi_slopes[h] : 0.0f;
  const float c1 = p.scale * hs;
  const float sl = slope * (float)dil;  // bias per sub-sequence step
  float kq, ks, k0 = 0.f, sc_a = 0.f, sc_b = 0.f;
  if constexpr (SOFTCAP) {
    const float f = 2.0f * kLog2e / p.softcap;
    kq = c1 * f;
    ks = sl * f;
    if constexpr (NORM == NORM_SOFTMAX) {
      sc_a = -2.0f * p.softcap * kLog2e;
      sc_b = p.softcap * kLog2e;
    } else if constexpr (NORM == NORM_SIGMOID) {
      sc_a = 2.0f * p.softcap * kLog2e;
      sc_b = -(p.softcap + p.bias) * kLog2e;
    } else {
      sc_a = -2.0f * p.softcap;
      sc_b = p.softcap;
    }
  } else if constexpr (NORM == NORM_SOFTMAX) {
    kq = c1 * kLog2e;
    ks = sl * kLog2e;
  } else if constexpr (NORM == NORM_SIGMOID) {
    kq = -c1 * kLog2e;
    ks = -sl * kLog2e;
    k0 = -p.bias * kLog2e;
  } else {
    kq = ALIBI ? c1 : 1.0f;  // without a bias the scale is applied to O instead
    ks = sl;
  }
  const float post = kRawRelu ? p.post_scale * c1 : p.post_scale;

  // ---- wavefront rows, Q fragments, per-row key intervals -------------------
  const int iw0 = q0 + wave * QW;
  const bool wave_valid = iw0 < g.S;
  const int wa = iw0, wb = imin32(iw0 + QW - 1, g.S - 1);

  bf16x8_t qf[QB][DK];
  int jl[QB], jh[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int i = iw0 + 32 * qb + lq;
    const bool ok = i < g.S;
    jl[qb] = key_lo(g, i);
    jh[qb] = key_hi(g, i);
    const uint16_t* src = qh + (int64_t)(ok ? i : 0) * qrs + 8 * lh;
#pragma unroll
    for (int kk = 0; kk < DK; ++kk) {
      u32x4_t val = *(const u32x4_t*)(src + 16 * kk);
      if (!ok) val = u32x4_t{0u, 0u, 0u, 0u};
      qf[qb][kk] = __builtin_bit_cast(bf16x8_t, val);
    }
  }

  // ---- KV tiles this workgroup visits ---------------------------------------
  const TileRange tr = tile_range(g, q0, imin32(q0 + BM - 1, g.S - 1), BN);
  const int ntiles = tr.n_pre + tr.n2;

  // Global -> VGPR -> LDS staging.  Thread t moves chunks c = t + 256 n of each
  // tile (row c / DQ, chunk c % DQ); rows past the end re-read the last row
  // (finite values; the mask gives their scores p = 0).
  u32x4_t kreg[NLD], vreg[NLD];
  auto load_tile = [&](int jt0) {
#pragma unroll
    for (int n = 0; n < NLD; ++n) {
      const int c = tid + kThreads * n;
      const int row = c / DQ, ch = c % DQ;
      const int j = imin32(jt0 + row, g.S - 1);
      kreg[n] = *(const u32x4_t*)(kh + (int64_t)j * krs + 8 * ch);
      vreg[n] = *(const u32x4_t*)(vh + (int64_t)j * vrs + 8 * ch);
    }
  };
  auto store_tile = [&](int stage) {
    char* ks_ = lds + stage * STAGE_BYTES;
    char* vs_ = ks_ + K_BYTES;
#pragma unroll
    for (int n = 0; n < NLD; ++n) {
      const int c = tid + kThreads * n;
      const int row = c / DQ, ch = c % DQ;
      *(u32x4_t*)(ks_ + row * KP + 16 * ch) = kreg[n];
      *(u32x4_t*)(vs_ + row * VP + 16 * ch) = vreg[n];
    }
  };

  // ---- accumulators ---------------------------------------------------------
  f32x16_t oacc[DB][QB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int e = 0; e < 16; ++e) oacc[db][qb][e] = 0.f;
  float m_run[QB], l_run[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m_run[qb] = -INFINITY;
    l_run[qb] = 0.f;
  }

  // Per-lane LDS byte offsets; every fragment is at a compile-time distance.
  // K fragment (kb, kk): row 32 kb + lq, elements 16 kk + 8 lh .. +7.
  const int k_lane = lq * KP + 16 * lh;
  // V transposed read (c, rr, db): lane (group g16, slot s16) addresses row
  // 16 c + 8 rr + 4 (g16 / 2) + s16 / 4, elements 32 db + 16 (g16 % 2) + 4 (s16 % 4) .. +3.
  const int g16 = lane >> 4, s16 = lane & 15;
  const int v_lane = K_BYTES + (4 * (g16 >> 1) + (s16 >> 2)) * VP + 2 * (16 * (g16 & 1) + 4 * (s16 & 3));

  // One 32-key block of one tile for this wavefront.
  auto key_block = [&](const char* St, int jt0, int kb, bool masked) {
    f32x16_t sacc[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int e = 0; e < 16; ++e) sacc[qb][e] = 0.f;

    // S^T = K Q^T for keys 32 kb .. 32 kb + 31
#pragma unroll
    for (int kk = 0; kk < DK; ++kk) {
      const bf16x8_t a = *(const bf16x8_t*)(St + k_lane + (32 * kb * KP + 32 * kk));
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
        sacc[qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[qb][kk], sacc[qb], 0, 0, 0);
    }

    // score modifier -> t (in place)
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      if constexpr (!kPlainSoftmax && !kRawRelu) {
        const int i = iw0 + 32 * qb + lq;
        const int jbase = jt0 + 32 * kb + 4 * lh;
        const float ksb = ALIBI ? ks * (float)(jbase - i) + k0 : k0;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int rc = 8 * (e >> 2) + (e & 3);  // key offset of register e
          const float qk = sacc[qb][e];
          float lin;
          if constexpr (ALIBI) lin = __builtin_fmaf(qk, kq, __builtin_fmaf(ks, (float)rc, ksb));
          else if constexpr (NORM == NORM_SIGMOID && !SOFTCAP) lin = __builtin_fmaf(qk, kq, k0);
          else lin = qk * kq;
          if constexpr (SOFTCAP) {
            const float u = __builtin_amdgcn_exp2f(lin);
            sacc[qb][e] = __builtin_fmaf(__builtin_amdgcn_rcpf(1.0f + u), sc_a, sc_b);
          } else {
            sacc[qb][e] = lin;
          }
        }
      }
    }
    // mask (PARTIAL tiles only): softmax/ReLU -> -inf, sigmoid input -> +inf; all give p = 0
    if (masked) {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        const int jbase = jt0 + 32 * kb + 4 * lh;
        const int vlo = jl[qb] - jbase, vhi = jh[qb] - jbase, vpre = g.prefix - jbase;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int rc = 8 * (e >> 2) + (e & 3);
          const bool vis = (rc < vpre) | ((rc >= vlo) & (rc <= vhi));
          sacc[qb][e] = vis ? sacc[qb][e] : ((NORM == NORM_SIGMOID) ? INFINITY : -INFINITY);
        }
      }
    }

    // normaliser -> p, packed to bf16 pairs (pk[qb][w] holds registers 2w, 2w+1)
    uint32_t pk[QB][8];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      if constexpr (NORM == NORM_SOFTMAX) {
        float mx = sacc[qb][0];
#pragma unroll
        for (int e = 1; e < 16; ++e) mx = fmaxf(mx, sacc[qb][e]);
        mx = xhalf_max(mx);
        if constexpr (kPlainSoftmax) mx = mx * kq;  // kq > 0
        const float m_old = m_run[qb];
        const float m_new = (mx > m_old + kRescaleLog2) ? mx : m_old;
        if (__any(m_new != m_old)) {
          const float alpha = (m_old == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_old - m_new);
          l_run[qb] *= alpha;
#pragma unroll
          for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int e = 0; e < 16; ++e) oacc[db][qb][e] *= alpha;
        }
        m_run[qb] = m_new;
        const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
        float ls = l_run[qb];
#pragma unroll
        for (int w = 0; w < 8; ++w) {
          float p0, p1;
          if constexpr (kPlainSoftmax) {
            p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[qb][2 * w], kq, -m_use));
            p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[qb][2 * w + 1], kq, -m_use));
          } else {
            p0 = __builtin_amdgcn_exp2f(sacc[qb][2 * w] - m_use);
            p1 = __builtin_amdgcn_exp2f(sacc[qb][2 * w + 1] - m_use);
          }
          const bf16x2_t pb = pack2(p0, p1);
          ls = __builtin_amdgcn_fdot2_f32_bf16(pb, kOnes2, ls, false);  // row sum of the bf16 weights
          pk[qb][w] = __builtin_bit_cast(uint32_t, pb);
        }
        l_run[qb] = ls;
      } else {
#pragma unroll
        for (int w = 0; w < 8; ++w) {
          float p0 = sacc[qb][2 * w], p1 = sacc[qb][2 * w + 1];
          if constexpr (NORM == NORM_SIGMOID) {
            p0 = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(p0));
            p1 = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(p1));
          } else {
            p0 = fmaxf(p0, 0.f);
            p1 = fmaxf(p1, 0.f);
          }
          pk[qb][w] = __builtin_bit_cast(uint32_t, pack2(p0, p1));
        }
      }
    }

    // O^T += V^T P^T over the two 16-key chunks of this block
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int c = 2 * kb + half;
      bf16x8_t pf[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        const u32x4_t w = {pk[qb][4 * half], pk[qb][4 * half + 1], pk[qb][4 * half + 2], pk[qb][4 * half + 3]};
        pf[qb] = __builtin_bit_cast(bf16x8_t, w);
      }
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const char* vp = St + v_lane + (16 * c * VP + 64 * db);
        const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)vp);
        const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(vp + 8 * VP));
        typedef short i16x8_t __attribute__((ext_vector_type(8)));
        const i16x8_t av = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        const bf16x8_t a = __builtin_bit_cast(bf16x8_t, av);
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
          oacc[db][qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pf[qb], oacc[db][qb], 0, 0, 0);
      }
    }
  };

  auto tile_step = [&](const char* St, int jt0, bool masked) {
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) key_block(St, jt0, kb, masked);
  };

  // ---- main loop: double-buffered LDS, one barrier per tile -----------------
  if (ntiles > 0) {
    load_tile(tile_at(tr, 0) * BN);
    store_tile(0);
  }
  __syncthreads();
  for (int it = 0; it < ntiles; ++it) {
    const int jt0 = tile_at(tr, it) * BN;
    const bool has_next = it + 1 < ntiles;
    if (has_next) load_tile(tile_at(tr, it + 1) * BN);
    const char* St = lds + (it & 1) * STAGE_BYTES;
    const int cls = wave_valid ? classify_tile(g, wa, wb, jt0, jt0 + BN - 1) : (int)TILE_EMPTY;
    if (cls != TILE_EMPTY) tile_step(St, jt0, cls == TILE_PARTIAL);
    if (has_next) store_tile((it + 1) & 1);
    __syncthreads();
  }

  // ---- epilogue: normalise and store ----------------------------------------
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int i = iw0 + 32 * qb + lq;
    float f;
    if constexpr (NORM == NORM_SOFTMAX) {
      const float lt = xhalf_sum(l_run[qb]);
      f = lt > 0.f ? 1.0f / lt : 0.f;
    } else {
      f = post;
    }
    if (i < g.S) {
      uint16_t* dst = oh + (int64_t)i * ors + 4 * lh;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          u32x2_t w;
          w[0] = pack_bf16x2(oacc[db][qb][4 * gq + 0] * f, oacc[db][qb][4 * gq + 1] * f);
          w[1] = pack_bf16x2(oacc[db][qb][4 * gq + 2] * f, oacc[db][qb][4 * gq + 3] * f);
          *(u32x2_t*)(dst + 32 * db + 8 * gq) = w;
        }
    }
  }
}

}  // namespace chia
