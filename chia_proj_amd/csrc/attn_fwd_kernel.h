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
//     (prefix tiles + the band hull), double-buffered through LDS with one
//     barrier per tile; each wavefront classifies the tile against its own
//     rows and skips it (EMPTY), runs it unmasked (FULL) or with the
//     per-element predicate (PARTIAL).
//
// Matrix-core formulation (v_mfma_f32_32x32x16_bf16, fp32 accumulate)
//   S^T[key, query] = K Q^T : A = K rows from LDS, B = Q rows kept in VGPRs.
//     The 32x32 accumulator gives each lane ONE query column and 16 keys, so
//     the softmax row max / row sum are in-lane reductions plus a single
//     exchange with lane^32.
//   O^T[d, query] += V^T P^T : the S^T accumulator registers, rounded to bf16,
//     are directly the B operand (lane = query, 8 keys).  The key order they
//     carry is {0-3, 8-11} (lanes 0-31) / {4-7, 12-15} (lanes 32-63) within
//     each 16-key chunk, so V is stored transposed in LDS with that same key
//     permutation and each A fragment is one 16-byte LDS read.
//   Online softmax runs in the exp2 domain with a lazily updated reference
//   max: the running max is only moved (and O, l rescaled) when a tile's max
//   exceeds it by more than kRescaleLog2, so p <= 2^kRescaleLog2.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mask.h"

namespace chia {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

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

// Queries per wavefront (in units of 32) for each head dim.
template <int D>
struct TileCfg {
  static constexpr int QB = (D == 64) ? 2 : 1;
};

// 16-byte-chunk XOR swizzle for LDS rows: 8 consecutive rows read the same
// logical chunk from 8 different bank groups.
__device__ __forceinline__ int swz(int chunk, int row) { return chunk ^ ((row ^ (row >> 3)) & 7); }

// Physical key (0..15 within a 16-key chunk) -> position in the permuted V^T
// order {0-3, 8-11, 4-7, 12-15} that matches the S^T accumulator layout.
__device__ __forceinline__ int vt_pos(int key) {
  const int w = key & 15, base = key & ~15;
  const int p = (w >= 4 && w < 8) ? w + 4 : ((w >= 8 && w < 12) ? w - 4 : w);
  return base + p;
}

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

template <bool B>
struct BoolTag {
  static constexpr bool value = B;
};

__device__ __forceinline__ float xhalf(float x) { return __shfl_xor(x, 32, 64); }

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const __bf16 x = (__bf16)a, y = (__bf16)b;
  return (uint32_t)__builtin_bit_cast(uint16_t, x) | ((uint32_t)__builtin_bit_cast(uint16_t, y) << 16);
}

template <int D, int QB, int NORM, bool ALIBI, bool SOFTCAP>
__global__ __launch_bounds__(kThreads) void attn_fwd_kernel(const FwdParams p) {
  constexpr int BN = kBN;
  constexpr int QW = 32 * QB;        // query rows per wavefront
  constexpr int BM = kWaves * QW;    // query rows per workgroup
  constexpr int KB = BN / 32;        // 32-key blocks per tile
  constexpr int DK = D / 16;         // k-steps of the QK^T MFMA
  constexpr int DB = D / 32;         // 32-row d blocks of O^T
  constexpr int NCH = BN / 16;       // 16-key chunks of the PV MFMA
  constexpr int DQ = D / 8;          // 16-byte chunks per K/V row
  constexpr int NK = BN * DQ / kThreads;        // K chunks per thread
  constexpr int NV = (BN / 2) * DQ / kThreads;  // V key-pair units per thread
  constexpr int K_ELEMS = BN * D;
  constexpr int STAGE = 2 * BN * D;  // K tile + V^T tile (u16 elements)
  static_assert(NK >= 1 && NV >= 1, "tile too small for the workgroup");
  constexpr bool kPlainSoftmax = (NORM == NORM_SOFTMAX) && !ALIBI && !SOFTCAP;

  __shared__ __attribute__((aligned(16))) uint16_t lds[2 * STAGE];

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
  const float post = (NORM == NORM_RELU && !ALIBI && !SOFTCAP) ? p.post_scale * c1 : p.post_scale;

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

  u32x4_t kreg[NK];
  u32x4_t vreg[NV][2];

  auto load_tile = [&](int jt0) {
#pragma unroll
    for (int n = 0; n < NK; ++n) {
      const int c = tid + kThreads * n;
      const int key = c / DQ, ch = c % DQ;
      const int j = jt0 + key;
      kreg[n] = (j < g.S) ? *(const u32x4_t*)(kh + (int64_t)j * krs + 8 * ch) : u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int n = 0; n < NV; ++n) {
      const int u = tid + kThreads * n;
      const int kp = u / DQ, ch = u % DQ;
      const int j = jt0 + 2 * kp;
      vreg[n][0] = (j < g.S) ? *(const u32x4_t*)(vh + (int64_t)j * vrs + 8 * ch) : u32x4_t{0u, 0u, 0u, 0u};
      vreg[n][1] = (j + 1 < g.S) ? *(const u32x4_t*)(vh + (int64_t)(j + 1) * vrs + 8 * ch)
                                 : u32x4_t{0u, 0u, 0u, 0u};
    }
  };

  auto store_tile = [&](int stage) {
    uint16_t* ks_ = lds + stage * STAGE;
    uint16_t* vs_ = ks_ + K_ELEMS;
#pragma unroll
    for (int n = 0; n < NK; ++n) {
      const int c = tid + kThreads * n;
      const int key = c / DQ, ch = c % DQ;
      *(u32x4_t*)(ks_ + key * D + 8 * swz(ch, key)) = kreg[n];
    }
#pragma unroll
    for (int n = 0; n < NV; ++n) {
      const int u = tid + kThreads * n;
      const int kp = u / DQ, ch = u % DQ;
      const int pos = vt_pos(2 * kp);  // even; key 2kp+1 sits right after it
      const int pch = pos >> 3, pin = pos & 7;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t a = vreg[n][0][e >> 1], bb = vreg[n][1][e >> 1];
        const uint32_t word = (e & 1) ? ((a >> 16) | (bb & 0xffff0000u)) : ((a & 0xffffu) | (bb << 16));
        const int d = 8 * ch + e;
        *(uint32_t*)(vs_ + d * BN + 8 * swz(pch, d) + pin) = word;
      }
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

  // One KV tile for this wavefront.  MASKED selects the per-element predicate.
  auto tile_step = [&](const uint16_t* Ks, const uint16_t* Vs, int jt0, auto masked_tag) {
    constexpr bool MASKED = decltype(masked_tag)::value;
    f32x16_t sacc[KB][QB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int e = 0; e < 16; ++e) sacc[kb][qb][e] = 0.f;

    // S^T = K Q^T
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const int key = 32 * kb + lq;
#pragma unroll
      for (int kk = 0; kk < DK; ++kk) {
        const bf16x8_t a = *(const bf16x8_t*)(Ks + key * D + 8 * swz(2 * kk + lh, key));
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
          sacc[kb][qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[qb][kk], sacc[kb][qb], 0, 0, 0);
      }
    }

    // score modifier, mask, normaliser
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int i = iw0 + 32 * qb + lq;
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const int jbase = jt0 + 32 * kb + 4 * lh;
        const int vlo = jl[qb] - jbase, vhi = jh[qb] - jbase, vpre = g.prefix - jbase;
        const float ksb = ALIBI ? ks * (float)(jbase - i) + k0 : k0;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int rc = 8 * (e >> 2) + (e & 3);  // key offset of register e
          const float qk = sacc[kb][qb][e];
          float t;
          if constexpr (kPlainSoftmax || (NORM == NORM_RELU && !ALIBI && !SOFTCAP)) {
            t = qk;
          } else {
            float lin;
            if constexpr (ALIBI) lin = __builtin_fmaf(qk, kq, __builtin_fmaf(ks, (float)rc, ksb));
            else if constexpr (NORM == NORM_SIGMOID && !SOFTCAP) lin = __builtin_fmaf(qk, kq, k0);
            else lin = qk * kq;
            if constexpr (SOFTCAP) {
              const float u = __builtin_amdgcn_exp2f(lin);
              t = __builtin_fmaf(__builtin_amdgcn_rcpf(1.0f + u), sc_a, sc_b);
            } else {
              t = lin;
            }
          }
          if constexpr (MASKED) {
            // masked entries: softmax/ReLU -> -inf, sigmoid input -> +inf; all give p = 0
            const bool vis = (rc < vpre) || (rc >= vlo && rc <= vhi);
            if (!vis) t = (NORM == NORM_SIGMOID) ? INFINITY : -INFINITY;
          }
          if constexpr (NORM == NORM_SOFTMAX) mx = fmaxf(mx, t);
          sacc[kb][qb][e] = t;
        }
      }

      if constexpr (NORM == NORM_SOFTMAX) {
        mx = fmaxf(mx, xhalf(mx));
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
        float ls = 0.f;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const float t = sacc[kb][qb][e];
            const float pe = kPlainSoftmax ? __builtin_amdgcn_exp2f(__builtin_fmaf(t, kq, -m_use))
                                           : __builtin_amdgcn_exp2f(t - m_use);
            ls += pe;
            sacc[kb][qb][e] = pe;
          }
        l_run[qb] += ls;
      } else {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const float t = sacc[kb][qb][e];
            float pe;
            if constexpr (NORM == NORM_SIGMOID) pe = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t));
            else pe = fmaxf(t, 0.f);
            sacc[kb][qb][e] = pe;
          }
      }
    }

    // O^T += V^T P^T
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      const int kb = c >> 1, half = c & 1;
      bf16x8_t pf[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        u32x4_t w;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          w[e] = pack_bf16x2(sacc[kb][qb][8 * half + 2 * e], sacc[kb][qb][8 * half + 2 * e + 1]);
        pf[qb] = __builtin_bit_cast(bf16x8_t, w);
      }
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const int d = 32 * db + lq;
        const bf16x8_t a = *(const bf16x8_t*)(Vs + d * BN + 8 * swz(2 * c + lh, d));
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
          oacc[db][qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pf[qb], oacc[db][qb], 0, 0, 0);
      }
    }
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
    const uint16_t* Ks = lds + (it & 1) * STAGE;
    const uint16_t* Vs = Ks + K_ELEMS;
    const int cls = wave_valid ? classify_tile(g, wa, wb, jt0, jt0 + BN - 1) : (int)TILE_EMPTY;
    if (cls == TILE_FULL) tile_step(Ks, Vs, jt0, BoolTag<false>{});
    else if (cls == TILE_PARTIAL) tile_step(Ks, Vs, jt0, BoolTag<true>{});
    if (has_next) store_tile((it + 1) & 1);
    __syncthreads();
  }

  // ---- epilogue: normalise and store ----------------------------------------
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int i = iw0 + 32 * qb + lq;
    float f;
    if constexpr (NORM == NORM_SOFTMAX) {
      const float lt = l_run[qb] + xhalf(l_run[qb]);
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
