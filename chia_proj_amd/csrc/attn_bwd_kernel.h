// attn_bwd_kernel.h -- gfx950 backward of the attention core: dQ, dK, dV.
//
// Semantics: the gradient of the forward in attn_fwd_kernel.h with respect to
// q, k and v (per-head scale, ALiBi slopes and the softcap are constants).
// Per score, with u = (q.k) c1 + slope (j - i), t = softcap tanh(u / softcap)
// (or u), p the normaliser's output and dp = do.v:
//   softmax  p = exp(t - lse_i),            dt = p (dp - delta_i),
//            delta_i = do_i . o_i
//   sigmoid  p = post sigma(t + bias),      dt = dp post sigma (1 - sigma)
//   ReLU     p = post max(t, 0),            dt = dp post [t > 0]
//   ds = dt (dt/du) c1,  dt/du = 1 - tanh^2 with a softcap, else 1
//   dV_j = sum_i p_ij do_i,  dK_j = sum_i ds_ij q_i,  dQ_i = sum_j ds_ij k_j
// Masked pairs have p = ds = 0.  The reference is forward-only; this follows
// the textbook derivation (autograd of the same formula is the oracle).
//
// Two launches, no atomics:
//   * attn_bwd_dq_kernel: a workgroup owns 128 query rows (32 per wavefront)
//     and streams the K / V tiles of their key range -- the forward's layout:
//     S^T = K Q^T and dP^T = V dO^T with Q, dO in registers, dS^T from the
//     lane's row statistics, dQ^T += K^T dS^T with K read transposed.  With
//     softmax it first computes its rows' statistics (lse log2 e and
//     delta = do . o) and stores them, negated delta, into a workspace laid
//     out per dilation residue (contiguous rows) for the second kernel;
//   * attn_bwd_dkdv_kernel: a workgroup owns 128 keys (32 per wavefront) of
//     one K/V head and streams the Q / dO tiles of the rows that see them, for
//     every query head of the group (GQA): S = Q K^T and dP = dO V^T with K, V
//     in registers (lane = key), dV^T += dO^T P and dK^T += Q^T dS with Q and
//     dO read transposed.
// Tiles are 64 rows, DMA'd HBM -> LDS as in the forward (one swizzle for both
// the row and the transposed reads), three LDS stages, one barrier per tile.
#pragma once
#include "attn_fwd_kernel.h"

namespace chia {

typedef float f32x4_t __attribute__((ext_vector_type(4)));

// 4-byte-per-lane HBM -> LDS DMA (uniform base + per-lane byte offset; lane l
// lands at lds_base + 4 l), ordered by the kernel's own vmcnt waits like
// dma16s.
__device__ __forceinline__ void dma4s(const void* sbase, uint32_t voff, uint32_t lds_base) {
  const uint64_t v = (uint64_t)(uintptr_t)sbase;
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
  const uint64_t u = ((uint64_t)hi << 32) | (uint64_t)lo;
  asm volatile("global_load_lds_dword %0, %1" ::"v"(voff), "s"(u), "{m0}"(lds_base) : "memory");
}

struct BwdParams {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint16_t* o;
  const uint16_t* dout;
  uint16_t* dq;
  uint16_t* dk;
  uint16_t* dv;
  int64_t q_sb, q_sh, q_ss;  // element strides: batch, head, seq
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int64_t do_sb, do_sh, do_ss;
  int64_t dq_sb, dq_sh, dq_ss;
  int64_t dk_sb, dk_sh, dk_ss;
  int64_t dv_sb, dv_sh, dv_ss;
  const float* lse;     // softmax: natural log, strides lse_sb / lse_sh / lse_ss
  int64_t lse_sb, lse_sh, lse_ss;
  const int32_t* cu_seqlens;  // packed sequences: [B + 1] token offsets, or nullptr
  const int32_t* seq_order;   // packed sequences: dispatch order of the B sequences, or nullptr
  float* stats;         // softmax: [B, H, R, SR] lse log2 e, then [B, H, R, SR] -delta
  const float* head_scale;
  const float* alibi_slopes;
  MaskSpec mask;
  int32_t B, H, G;      // G: query heads per K/V head
  int32_t residues, SR;  // SR: stats row stride (residue 0 length, padded)
  int32_t n_blk, n_wg;  // 128-row (or key) blocks per (b, head, residue 0); grid
  UDiv div_blk, div_res, div_h, div_g, div_hk, div_dil;
  float scale, softcap, bias, post_scale;
  // Causal rows: the launched kernel's slices per XCD for the longest-first
  // order (rank_order), 0 otherwise; and its divider.
  int32_t rank_hx;
  UDiv div_hx;
};

// Per-score gradient (see the header): from the raw s = q.k, dp = do.v and
// j - i, the probability p (for dV) and ds / c1 (for dQ, dK); the caller
// applies c1, once per accumulated gradient where it is uniform.  Softmax: the
// dP accumulator starts from -delta_i, so `dp` here is already dp - delta.
template <int NORM, bool ALIBI, bool SOFTCAP>
struct ScoreGrad {
  float c1, c1l2, sl, cap, k2cap, post, nbias_l2;
  float bq;  // sl / c1: the ALiBi bias per key step in units of q . k (accumulator seed)
  float c1k2;   // c1 * k2cap
  float capl2;  // cap * log2 e

  __device__ __forceinline__ void operator()(float s, float dp, float jmi, float lse2, float& p, float& ds) const {
    if constexpr (!ALIBI && !SOFTCAP) {
      // t = s c1: the scale folds into one fma ahead of the exponential
      if constexpr (NORM == NORM_SOFTMAX) {
        p = __builtin_amdgcn_exp2f(__builtin_fmaf(s, c1l2, -lse2));
        ds = p * dp;
      } else if constexpr (NORM == NORM_SIGMOID) {
        const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(__builtin_fmaf(s, -c1l2, nbias_l2)));
        p = post * sg;
        ds = dp * p * (1.0f - sg);
      } else {
        const float t = s * c1;
        p = post * fmaxf(t, 0.0f);
        ds = t > 0.0f ? dp * post : 0.0f;
      }
    } else {
      // u = s c1 (+ sl (j - i)); with softcap t = cap th, th = tanh(u / cap)
      // = 1 - 2 / (1 + 2^(2 u log2e / cap)), and the cap folds into the
      // exponent's fma
      float t, th = 0.0f, dtdu = 1.0f, uk = 0.0f;
      if constexpr (SOFTCAP) {
        uk = ALIBI ? __builtin_fmaf(sl, jmi, s * c1) * k2cap : s * c1k2;
        th = __builtin_fmaf(-2.0f, __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(uk)), 1.0f);
        dtdu = __builtin_fmaf(-th, th, 1.0f);
        t = cap * th;
      } else {
        t = ALIBI ? __builtin_fmaf(sl, jmi, s * c1) : s * c1;
      }
      float dt;
      if constexpr (NORM == NORM_SOFTMAX) {
        p = __builtin_amdgcn_exp2f(SOFTCAP ? __builtin_fmaf(th, capl2, -lse2) : __builtin_fmaf(t, kLog2e, -lse2));
        dt = p * dp;
      } else if constexpr (NORM == NORM_SIGMOID) {
        const float z = SOFTCAP ? __builtin_fmaf(-th, capl2, nbias_l2) : __builtin_fmaf(-t, kLog2e, nbias_l2);
        const float sg = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(z));
        p = post * sg;
        dt = dp * p * (1.0f - sg);
      } else {
        p = post * fmaxf(t, 0.0f);
        // [t > 0] = [u > 0], read from u: with softcap, 1 - 2 / (1 + 2^uk)
        // cancels to exactly 0 for |uk| below about 2^-24, which would drop
        // the whole derivative of such a score
        dt = (SOFTCAP ? uk : t) > 0.0f ? dp * post : 0.0f;
      }
      ds = dt * dtdu;
    }
  }

  __device__ __forceinline__ void set_head(float c1_, float sl_) {
    c1 = c1_;
    c1l2 = c1_ * kLog2e;
    sl = sl_;
    bq = sl_ / c1_;
    c1k2 = c1_ * k2cap;
  }
};

// Zero the elements of x[16] whose bit rc(e) = 8 (e >> 2) + (e & 3) is set in
// `hidden` (v_bfe_i32 + one bitwise blend per element, no compare / select).
__device__ __forceinline__ void zero_hidden(float* x, uint32_t hidden) {
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    uint32_t m = (uint32_t)__builtin_amdgcn_sbfe((int)hidden, 8 * (e >> 2) + (e & 3), 1);
    asm("" : "+v"(m));  // keeps the and-not bitwise
    x[e] = __uint_as_float(__float_as_uint(x[e]) & ~m);
  }
}

// The per-call constants (no memory access); c1 and sl are the query head's
// scale * head_scale and ALiBi slope per sub-sequence step, set by the caller.
template <int NORM, bool ALIBI, bool SOFTCAP>
__device__ __forceinline__ ScoreGrad<NORM, ALIBI, SOFTCAP> score_consts(const BwdParams& p) {
  ScoreGrad<NORM, ALIBI, SOFTCAP> f;
  f.cap = p.softcap;
  f.k2cap = SOFTCAP ? 2.0f * kLog2e / p.softcap : 0.0f;
  f.capl2 = p.softcap * kLog2e;
  f.post = p.post_scale;
  f.nbias_l2 = -p.bias * kLog2e;
  f.set_head(p.scale, 0.0f);
  return f;
}

// One 64-row tile of a [S, D] bf16 tensor (row stride rs elements, rows from
// `row` of the residue's sub-sequence, clamped to S - 1) into LDS at `dst`:
// row r, 16-byte chunk c lands in slot k_slot<D>(r, c), which keeps both the
// row reads and the transposed reads of the tile free of bank conflicts.
// Wavefront w of NW moves
// chunks [(n NW + w) 64, +64) for n < NDMA.
template <int D, int NW>
__device__ __forceinline__ void dma_rows(const uint16_t* base, int64_t rs, int row, int S, char* dst, int wave,
                                         int lane) {
  constexpr int DQ = D / 8;
  constexpr int NDMA = 64 * DQ / (NW * 64);
  const uint16_t* src = base + (int64_t)row * rs;
#pragma unroll
  for (int n = 0; n < NDMA; ++n) {
    const int pos = (n * NW + wave) * 64 + lane;
    const int r = pos / DQ, slot = pos % DQ;
    const int rr = imin32(r, S - 1 - row);
    dma16s(src, (uint32_t)(2 * ((int64_t)rr * rs + 8 * k_slot<D>(r, slot))), lds_addr(dst + (n * NW + wave) * 1024));
  }
}

// dma_rows with its per-lane offsets computed once for a fixed row stride: a
// tile whose 64 rows lie inside the sub-sequence adds only its uniform row
// base, a 32 x 32 -> 64-bit product (rows are non-negative and a row step is
// below 2^25 elements, so its byte count fits 32 bits); the last tile, whose
// rows past the end are clamped, takes dma_rows.
template <int D, int NW>
struct RowDma {
  static constexpr int DQ = D / 8, NDMA = 64 * DQ / (NW * 64);
  uint32_t off[NDMA];
  uint32_t row_bytes;
  __device__ RowDma(int64_t rs, int wave, int lane) : row_bytes(2u * (uint32_t)rs) {
#pragma unroll
    for (int n = 0; n < NDMA; ++n) {
      const int pos = (n * NW + wave) * 64 + lane;
      const int r = pos / DQ, slot = pos % DQ;
      off[n] = (uint32_t)r * row_bytes + 16 * k_slot<D>(r, slot);
    }
  }
  __device__ void operator()(const uint16_t* base, int64_t rs, int row, int S, char* dst, int wave, int lane) const {
    if (row + 64 <= S) {
      const uint16_t* src = (const uint16_t*)((const char*)base + (uint64_t)(uint32_t)row * row_bytes);
#pragma unroll
      for (int n = 0; n < NDMA; ++n) dma16s(src, off[n], lds_addr(dst + (n * NW + wave) * 1024));
    } else {
      dma_rows<D, NW>(base, rs, row, S, dst, wave, lane);
    }
  }
};

// The stage of tile it + NS - 1 (the DMA's, one iteration ahead of the
// compute's stage `cur` = it mod NS): without a division when NS is not a
// power of two.
template <int NS>
__device__ __forceinline__ uint32_t stage_behind(uint32_t cur) {
  return cur == 0 ? NS - 1 : cur - 1;
}

// Kernel set of one (head_dim, normaliser, ALiBi, softcap) instantiation.
using BwdKernelFn = void (*)(BwdParams);
struct BwdKernels {
  BwdKernelFn dq, dkdv, dkdv_head_c1;  // dkdv_head_c1: a group's heads differ in scale
};

// do . o over the 8 DK bf16 values of one lane's half row (chunks 16 kk + 8 lh
// of the dQ kernel's register layout), in fp32.
template <int DK>
__device__ __forceinline__ float half_row_dot(const bf16x8_t* x, const bf16x8_t* y) {
  float acc = 0.f;
#pragma unroll
  for (int kk = 0; kk < DK; ++kk) {
    const u32x4_t a = __builtin_bit_cast(u32x4_t, x[kk]), b = __builtin_bit_cast(u32x4_t, y[kk]);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      acc = __builtin_fmaf(__uint_as_float(a[w] << 16), __uint_as_float(b[w] << 16), acc);
      acc = __builtin_fmaf(__uint_as_float(a[w] & 0xffff0000u), __uint_as_float(b[w] & 0xffff0000u), acc);
    }
  }
  return acc;
}


// ---- dQ ------------------------------------------------------------------------
template <int D, int NORM, bool ALIBI, bool SOFTCAP>
__global__ __launch_bounds__(256, D == 64 ? 2 : 1) void attn_bwd_dq_kernel(const BwdParams p) {
  constexpr int NW = 4, BN = 64, KB = BN / 32, DK = D / 16, DB = D / 32;
  constexpr int RP = 2 * D, T_BYTES = BN * RP, STAGE_BYTES = 2 * T_BYTES;
  constexpr int NS = 3;
  __shared__ __attribute__((aligned(1024))) char lds[NS * STAGE_BYTES];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane & 31, lh = lane >> 5;

  // workgroup -> (b, h, residue, 128-row block), heaviest blocks first
  // (packed sequences of unequal length: round-robin over the XCDs, no remap)
  // the query blocks with the most keys first
  int bhr, blk;
  if (p.rank_hx > 0) {
    const SliceUnit su = rank_order((int)blockIdx.x, p.rank_hx, p.div_hx, p.n_blk);
    bhr = su.slice;
    blk = su.unit;
  } else {
    const int L = p.cu_seqlens ? (int)blockIdx.x : xcd_remap(blockIdx.x, p.n_wg);
    bhr = udiv(L, p.div_blk);
    blk = p.n_blk - 1 - (L - bhr * p.n_blk);
  }
  const int bh = udiv(bhr, p.div_res), r = bhr - bh * p.residues;
  const int bs = udiv(bh, p.div_h), h = bh - bs * p.H;
  const int b = seq_of(p.seq_order, bs);
  const SeqSpan seq = seq_span(p.cu_seqlens, b, p.mask.S);
  MaskSpec ms = p.mask;
  ms.S = seq.len;
  const MaskGeom g = residue_geom(ms, r);
  const int nblk_r = (g.S + 127) / 128;
  if (blk >= nblk_r) return;  // whole workgroup, before any barrier
  const int hkv = udiv(h, p.div_g);
  const int dil = p.mask.dil;
  const int64_t t0 = seq.tok0 + r;  // the residue's first token
  const uint16_t* qh = p.q + b * p.q_sb + h * p.q_sh + t0 * p.q_ss;
  const uint16_t* doh = p.dout + b * p.do_sb + h * p.do_sh + t0 * p.do_ss;
  const uint16_t* kh = p.k + b * p.k_sb + hkv * p.k_sh + t0 * p.k_ss;
  const uint16_t* vh = p.v + b * p.v_sb + hkv * p.v_sh + t0 * p.v_ss;
  uint16_t* dqh = p.dq + b * p.dq_sb + h * p.dq_sh + t0 * p.dq_ss;
  const int64_t qrs = p.q_ss * dil, dors = p.do_ss * dil, krs = p.k_ss * dil, vrs = p.v_ss * dil,
                dqrs = p.dq_ss * dil;
  // ALiBi without softcap seeds the S accumulator with the bias over c1 and
  // scores it with the plain (unbiased) formulas.
  constexpr bool kSeed = ALIBI && !SOFTCAP;
  ScoreGrad<NORM, ALIBI && !kSeed, SOFTCAP> sg = score_consts<NORM, ALIBI && !kSeed, SOFTCAP>(p);
  sg.set_head(p.scale * (p.head_scale ? p.head_scale[h] : 1.0f),
              (ALIBI && p.alibi_slopes) ? p.alibi_slopes[h] * (float)dil : 0.0f);

  // this wavefront's 32 rows: Q and dO as MFMA B operands (lane = row)
  const int row0 = blk * 128 + 32 * wave;
  const int i = row0 + lq;
  const bool ok = i < g.S;
  bf16x8_t qf[DK], df[DK];
  {
    const uint16_t* qs = qh + (int64_t)(ok ? i : 0) * qrs + 8 * lh;
    const uint16_t* ds = doh + (int64_t)(ok ? i : 0) * dors + 8 * lh;
#pragma unroll
    for (int kk = 0; kk < DK; ++kk) {
      qf[kk] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)(qs + 16 * kk));
      df[kk] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)(ds + 16 * kk));
    }
  }
  // softmax row statistics: the lane's half row of O, loaded beside Q and dO;
  // the row's lse and the arithmetic follow the DMA prologue
  bf16x8_t of[DK];
  float lse2 = 0.f, ndelta = 0.f;
  if constexpr (NORM == NORM_SOFTMAX) {
    const uint16_t* os = p.o + b * p.o_sb + h * p.o_sh + (t0 + (int64_t)(ok ? i : 0) * dil) * p.o_ss + 8 * lh;
#pragma unroll
    for (int kk = 0; kk < DK; ++kk) of[kk] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)(os + 16 * kk));
  }

  // key tiles of the workgroup's rows; per-wavefront classification bounds
  const int wg_hi = imin32(blk * 128 + 127, g.S - 1);
  const TileRange tr = tile_range(g, blk * 128, wg_hi, BN);
  const int ntiles = tr.n_pre + tr.n2;
  const bool wvalid = row0 < g.S;
  const int ra = row0, rb = imin32(row0 + 31, g.S - 1);

  f32x16_t dq[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) dq[db][e] = 0.f;

  // LDS lane offsets: row reads (A = K or V rows) and transposed reads (A = K^T)
  const int k_lane = lq * RP + 16 * k_slot<D>(lq, lh);
  const int g16 = lane >> 4, s16 = lane & 15;
  const int t_row = 4 * (g16 >> 1) + (s16 >> 2);
  const int t_lane = t_row * RP + 16 * k_slot<D>(t_row, 2 * (g16 & 1) + ((s16 & 3) >> 1)) + 8 * (s16 & 1);
  const int t_lane8 = (t_lane ^ (16 * row_swz<D>(8))) + 8 * RP;  // the same lanes 8 rows down

  // Scalar work per tile is kept small: a tile's first key is the previous
  // tile's plus BN except at the seam between prefix and band tiles (and the
  // first), separately for the DMA (NS - 1 tiles ahead) and the compute; the
  // stage is a wrapping counter; the class comes from per-wavefront bounds
  // (mask.h); the DMA's per-lane offsets are fixed once.
  const int seam = tr.n_pre;
  const RowDma<D, NW> kdma(krs, wave, lane), vdma(vrs, wave, lane);
  auto issue = [&](int jt0, uint32_t stage) {
    char* st = lds + stage * STAGE_BYTES;
    kdma(kh, krs, jt0, g.S, st, wave, lane);
    vdma(vh, vrs, jt0, g.S, st + T_BYTES, wave, lane);
  };
  constexpr int NDMA2 = 2 * (64 * (D / 8) / (NW * 64));  // loads per tile per wavefront
  int dma_next = 0, jt_dma = 0;
  for (; dma_next < NS - 1 && dma_next < ntiles; ++dma_next) {
    jt_dma = (dma_next == 0 || dma_next == seam) ? tile_at(tr, dma_next) * BN : jt_dma + BN;
    issue(jt_dma, (uint32_t)dma_next);
  }
  const KeyRanges<BN> kr(g, wvalid, ra, rb);
  int jt0 = 0;
  uint32_t st_cur = 0;
  // Q, dO and the row statistics in registers before the loop: otherwise the
  // compiler's waits for these loads sink into the loop, where their vmcnt
  // also drains the K/V tiles in flight (the compiler does not count the DMA)
#pragma unroll
  for (int kk = 0; kk < DK; ++kk) asm volatile("" : "+v"(qf[kk]), "+v"(df[kk]));
  if constexpr (NORM == NORM_SOFTMAX) {
    // lse log2 e, and -delta (the dP accumulators' seed) from do . o: this
    // lane's half row, then its partner's (lane ^ 32); stored for dK/dV
    lse2 = p.lse[b * p.lse_sb + h * p.lse_sh + (t0 + (int64_t)(ok ? i : 0) * dil) * p.lse_ss] * kLog2e;
    const float part = half_row_dot<DK>(df, of);
    ndelta = -(part + __shfl_xor(part, 32));
    if (ok && lh == 0) {
      const int64_t o2 = ((int64_t)(b * p.H + h) * p.residues + r) * p.SR + i;  // b: the sequence
      p.stats[o2] = lse2;
      p.stats[(int64_t)p.B * p.H * p.residues * p.SR + o2] = ndelta;
    }
    asm volatile("" : "+v"(lse2), "+v"(ndelta));
  }

  typedef short i16x8_t __attribute__((ext_vector_type(8)));
  for (int it = 0; it < ntiles; ++it) {
    if (dma_next - (it + 1) >= 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NDMA2) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const uint32_t st_it = st_cur;  // it mod NS
    st_cur = st_it + 1 == NS ? 0 : st_it + 1;
    if (dma_next < ntiles) {
      jt_dma = dma_next == seam ? tile_at(tr, dma_next) * BN : jt_dma + BN;
      issue(jt_dma, stage_behind<NS>(st_it));
      ++dma_next;
    }
    const char* St = lds + st_it * STAGE_BYTES;
    jt0 = (it == 0 || it == seam) ? tile_at(tr, it) * BN : jt0 + BN;
    const int cls = key_class(kr, jt0);
    if (cls == TILE_EMPTY) continue;

    uint32_t pk[KB][8];  // dS^T, bf16 pairs
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      f32x16_t sacc, pacc;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        sacc[e] = 0.f;
        pacc[e] = NORM == NORM_SOFTMAX ? ndelta : 0.f;
      }
      if constexpr (kSeed) {  // register e: key jt0 + 32 kb + 4 lh + rc(e), query i
        const float b0 = sg.bq * (float)(jt0 + 32 * kb + 4 * lh - i);
#pragma unroll
        for (int e = 0; e < 16; ++e) sacc[e] = __builtin_fmaf(sg.bq, (float)(8 * (e >> 2) + (e & 3)), b0);
      }
#pragma unroll
      for (int kk = 0; kk < DK; ++kk) {
        const bf16x8_t a = *(const bf16x8_t*)(St + 32 * kb * RP + (k_lane ^ (32 * kk)));
        const bf16x8_t av = *(const bf16x8_t*)(St + T_BYTES + 32 * kb * RP + (k_lane ^ (32 * kk)));
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[kk], sacc, 0, 0, 0);
        pacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, df[kk], pacc, 0, 0, 0);
      }
      const int jbase = jt0 + 32 * kb + 4 * lh;
      float ds[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        float pv;
        sg(sacc[e], pacc[e], (float)(jbase + 8 * (e >> 2) + (e & 3) - i), lse2, pv, ds[e]);
      }
      if (cls == TILE_PARTIAL) zero_hidden(ds, hidden_bits(g, i, jbase));
#pragma unroll
      for (int w = 0; w < 8; ++w) pk[kb][w] = pack_bf16x2(ds[2 * w], ds[2 * w + 1]);
    }
    // dQ^T += K^T dS^T, 16-key chunk by chunk
#pragma unroll
    for (int c = 0; c < 2 * KB; ++c) {
      const int kb = c >> 1, half = c & 1;
#pragma unroll
      for (int db = 0; db < DB; ++db) {
        const char* ka = St + 16 * c * RP;
        const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(ka + (t_lane ^ (64 * db))));
        const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(ka + (t_lane8 ^ (64 * db))));
        const bf16x8_t a = __builtin_bit_cast(bf16x8_t, (i16x8_t)__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
        const u32x4_t wv = {pk[kb][4 * half], pk[kb][4 * half + 1], pk[kb][4 * half + 2], pk[kb][4 * half + 3]};
        dq[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, __builtin_bit_cast(bf16x8_t, wv), dq[db], 0, 0, 0);
      }
    }
  }

  if (ok) {
    // ds was accumulated without the head's scale
    const float c1 = sg.c1;
    uint16_t* dst = dqh + (int64_t)i * dqrs + 4 * lh;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        u32x2_t w;
        w[0] = pack_bf16x2(dq[db][4 * gq + 0] * c1, dq[db][4 * gq + 1] * c1);
        w[1] = pack_bf16x2(dq[db][4 * gq + 2] * c1, dq[db][4 * gq + 3] * c1);
        *(u32x2_t*)(dst + 32 * db + 8 * gq) = w;
      }
  }
}

// ---- dK, dV ----------------------------------------------------------------------
// HEAD_C1: the query heads of a K/V group differ in score scale (GQA with
// per-head scales), so c1 multiplies each score; otherwise it multiplies dK
// once at the store.
template <int D, int NORM, bool ALIBI, bool SOFTCAP, bool HEAD_C1>
__global__ __launch_bounds__(256, D == 64 ? 2 : 1) void attn_bwd_dkdv_kernel(const BwdParams p) {
  constexpr int NW = 4, BM = 64, QB = BM / 32, DK = D / 16, DB = D / 32;
  constexpr int RP = 2 * D, T_BYTES = BM * RP;
  // stage: Q tile, dO tile, then (softmax) the 64 rows' lse log2 e and -delta
  constexpr bool kStats = NORM == NORM_SOFTMAX;
  constexpr int STAGE_BYTES = 2 * T_BYTES + (kStats ? 512 : 0);
  constexpr int NS = 3;
  constexpr int kMaxGroup = 256;  // query heads per K/V head staged in LDS
  __shared__ __attribute__((aligned(1024))) char lds[NS * STAGE_BYTES];
  __shared__ float head_c[2 * kMaxGroup];  // per query head of the group: c1, ALiBi slope

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane & 31, lh = lane >> 5;

  // workgroup -> (b, K/V head, residue, 128-key block); low blocks (seen by
  // the most rows under a causal mask) first
  const int HK = p.H / p.G;
  // the key blocks with the most queries (the first ones) first
  int bhr, blk;
  if (p.rank_hx > 0) {
    const SliceUnit su = rank_order((int)blockIdx.x, p.rank_hx, p.div_hx, p.n_blk);
    bhr = su.slice;
    blk = p.n_blk - 1 - su.unit;
  } else {
    const int L = p.cu_seqlens ? (int)blockIdx.x : xcd_remap(blockIdx.x, p.n_wg);
    bhr = udiv(L, p.div_blk);
    blk = L - bhr * p.n_blk;
  }
  const int bh = udiv(bhr, p.div_res), r = bhr - bh * p.residues;
  const int bs = udiv(bh, p.div_hk), hkv = bh - bs * HK;
  const int b = seq_of(p.seq_order, bs);
  const SeqSpan seq = seq_span(p.cu_seqlens, b, p.mask.S);
  MaskSpec ms = p.mask;
  ms.S = seq.len;
  const MaskGeom g = residue_geom(ms, r);
  const int nblk_r = (g.S + 127) / 128;
  if (blk >= nblk_r) return;  // whole workgroup, before any barrier
  const int dil = p.mask.dil;
  const int64_t t0 = seq.tok0 + r;  // the residue's first token
  const uint16_t* kh = p.k + b * p.k_sb + hkv * p.k_sh + t0 * p.k_ss;
  const uint16_t* vh = p.v + b * p.v_sb + hkv * p.v_sh + t0 * p.v_ss;
  uint16_t* dkh = p.dk + b * p.dk_sb + hkv * p.dk_sh + t0 * p.dk_ss;
  uint16_t* dvh = p.dv + b * p.dv_sb + hkv * p.dv_sh + t0 * p.dv_ss;
  const int64_t qrs = p.q_ss * dil, dors = p.do_ss * dil, krs = p.k_ss * dil, vrs = p.v_ss * dil,
                dkrs = p.dk_ss * dil, dvrs = p.dv_ss * dil;

  // the group's per-head score constants, once, before any DMA is in flight
  for (int t = tid; t < p.G; t += NW * 64) {
    const int hq = hkv * p.G + t;
    head_c[t] = p.scale * (p.head_scale ? p.head_scale[hq] : 1.0f);
    head_c[kMaxGroup + t] = (ALIBI && p.alibi_slopes) ? p.alibi_slopes[hq] * (float)p.mask.dil : 0.0f;
  }
  __syncthreads();
  // ds leaves the score step without c1: applied to dK at the store when the
  // group shares one scale, else per score
  const float c1u = HEAD_C1 ? 1.0f : head_c[0];

  // this wavefront's 32 keys: K and V as MFMA B operands (lane = key)
  const int key0 = blk * 128 + 32 * wave;
  const int j = key0 + lq;
  const bool okj = j < g.S;
  bf16x8_t kf[DK], vf[DK];
  {
    const uint16_t* ks = kh + (int64_t)(okj ? j : 0) * krs + 8 * lh;
    const uint16_t* vs = vh + (int64_t)(okj ? j : 0) * vrs + 8 * lh;
#pragma unroll
    for (int kk = 0; kk < DK; ++kk) {
      kf[kk] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)(ks + 16 * kk));
      vf[kk] = __builtin_bit_cast(bf16x8_t, *(const u32x4_t*)(vs + 16 * kk));
    }
  }

  // query tiles of the rows that see the workgroup's keys, for each query head of the group
  const RowSpan qs = query_range(g, blk * 128, imin32(blk * 128 + 127, g.S - 1));
  const int t_lo = qs.lo / BM, n_qt = qs.lo <= qs.hi ? qs.hi / BM - t_lo + 1 : 0;
  const int ntiles = n_qt * p.G;
  const bool wvalid = key0 < g.S;
  const int kc = key0, kd = key0 + 31;
  // the rows that see this lane's key: an interval (exact for one key; empty
  // past the end), so a block's per-element mask is one bitmask per lane
  const RowSpan seen = query_range(g, j, j);
  const int64_t plane = (int64_t)p.B * p.H * p.residues * p.SR;

  f32x16_t dk[DB], dv[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) dk[db][e] = dv[db][e] = 0.f;

  const int k_lane = lq * RP + 16 * k_slot<D>(lq, lh);
  const int g16 = lane >> 4, s16 = lane & 15;
  const int t_row = 4 * (g16 >> 1) + (s16 >> 2);
  const int t_lane = t_row * RP + 16 * k_slot<D>(t_row, 2 * (g16 & 1) + ((s16 & 3) >> 1)) + 8 * (s16 & 1);
  const int t_lane8 = (t_lane ^ (16 * row_swz<D>(8))) + 8 * RP;  // the same lanes 8 rows down

  // Tiles run row tile t_lo .. t_lo + n_qt - 1 of query head hkv G, then of the
  // next head of the group.  Two cursors walk them (the DMA one runs ahead);
  // a head's base pointers are advanced only when the head changes.
  struct Cursor {
    int qt, hq;
    const uint16_t* qb;
    const uint16_t* dob;
    const float* sb;
  };
  auto cursor0 = [&]() {
    const int hq = hkv * p.G;
    return Cursor{t_lo, hq, p.q + b * p.q_sb + hq * p.q_sh + t0 * p.q_ss,
                  p.dout + b * p.do_sb + hq * p.do_sh + t0 * p.do_ss,
                  p.stats + ((int64_t)(b * p.H + hq) * p.residues + r) * p.SR};
  };
  auto advance = [&](Cursor& c) {
    if (++c.qt == t_lo + n_qt) {
      c.qt = t_lo;
      ++c.hq;
      c.qb += p.q_sh;
      c.dob += p.do_sh;
      c.sb += (int64_t)p.residues * p.SR;
    }
  };
  Cursor dc = cursor0(), cc = cursor0();
  // Scalar work per tile is kept small: the stage is a wrapping counter, the
  // class of a row tile comes from the wavefront's two row spans (mask.h), and
  // the DMA's per-lane offsets are fixed once.
  const RowDma<D, NW> qdma(qrs, wave, lane), dodma(dors, wave, lane);
  const RowRanges<BM> rr(g, wvalid, kc, kd);
  uint32_t st_cur = 0;
  auto issue = [&](uint32_t stage) {
    const int i0 = dc.qt * BM;
    char* st = lds + stage * STAGE_BYTES;
    qdma(dc.qb, qrs, i0, g.S, st, wave, lane);
    dodma(dc.dob, dors, i0, g.S, st + T_BYTES, wave, lane);
    if constexpr (kStats) {
      // wavefront w moves 32 floats: lse log2 e rows [32 w, +32) (w < 2), or
      // -delta rows [32 (w - 2), +32); the stats rows are padded to 64
      const float* src = dc.sb + (wave >= 2 ? plane : 0) + i0 + 32 * (wave & 1);
      if (lane < 32) dma4s(src, (uint32_t)(4 * lane), lds_addr(st + 2 * T_BYTES + 128 * wave));
    }
    advance(dc);
  };
  constexpr int NDMA2 = 2 * (64 * (D / 8) / (NW * 64)) + (kStats ? 1 : 0);
  int dma_next = 0;
  for (; dma_next < NS - 1 && dma_next < ntiles; ++dma_next) issue((uint32_t)dma_next);
  // K and V in registers before the loop (see the dQ kernel)
#pragma unroll
  for (int kk = 0; kk < DK; ++kk) asm volatile("" : "+v"(kf[kk]), "+v"(vf[kk]));

  typedef short i16x8_t __attribute__((ext_vector_type(8)));
  for (int it = 0; it < ntiles; ++it) {
    if (dma_next - (it + 1) >= 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NDMA2) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const uint32_t st_it = st_cur;  // it mod NS
    st_cur = st_it + 1 == NS ? 0 : st_it + 1;
    if (dma_next < ntiles) {
      issue(stage_behind<NS>(st_it));
      ++dma_next;
    }
    const char* St = lds + st_it * STAGE_BYTES;
    const int hq = cc.hq, i0 = cc.qt * BM;
    advance(cc);
    // rows past the end of the sub-sequence are clamped copies: mask them
    int cls = row_class(rr, i0);
    if (cls == TILE_EMPTY) continue;
    if (i0 + BM > g.S) cls = TILE_PARTIAL;
    constexpr bool kSeed = ALIBI && !SOFTCAP;  // as in the dQ kernel
    ScoreGrad<NORM, ALIBI && !kSeed, SOFTCAP> sg = score_consts<NORM, ALIBI && !kSeed, SOFTCAP>(p);
    sg.set_head(head_c[hq - hkv * p.G], head_c[kMaxGroup + hq - hkv * p.G]);
    const float* st_stats = (const float*)(St + 2 * T_BYTES);  // [64] lse log2 e, then [64] -delta

#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      // rows of register e: ibase + 8 (e >> 2) + (e & 3); softmax: their lse
      // log2 e, and -delta as the dP accumulator's seed
      const int ibase = i0 + 32 * qb + 4 * lh;
      f32x4_t l4[4], d4[4];
      if constexpr (kStats) {
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          l4[gq] = *(const f32x4_t*)(st_stats + 32 * qb + 4 * lh + 8 * gq);
          d4[gq] = *(const f32x4_t*)(st_stats + 64 + 32 * qb + 4 * lh + 8 * gq);
        }
      }
      f32x16_t sacc, pacc;
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        sacc[e] = 0.f;
        pacc[e] = kStats ? d4[e >> 2][e & 3] : 0.f;
      }
      if constexpr (kSeed) {  // register e: query i0 + 32 qb + 4 lh + rc(e), key j
        const float b0 = sg.bq * (float)(j - (i0 + 32 * qb + 4 * lh));
#pragma unroll
        for (int e = 0; e < 16; ++e) sacc[e] = __builtin_fmaf(-sg.bq, (float)(8 * (e >> 2) + (e & 3)), b0);
      }
#pragma unroll
      for (int kk = 0; kk < DK; ++kk) {
        const bf16x8_t a = *(const bf16x8_t*)(St + 32 * qb * RP + (k_lane ^ (32 * kk)));
        const bf16x8_t ad = *(const bf16x8_t*)(St + T_BYTES + 32 * qb * RP + (k_lane ^ (32 * kk)));
        sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, kf[kk], sacc, 0, 0, 0);
        pacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ad, vf[kk], pacc, 0, 0, 0);
      }
      float pv[16], dsv[16];
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int rc = 8 * (e >> 2) + (e & 3);
        const float ls = kStats ? l4[e >> 2][e & 3] : 0.f;
        sg(sacc[e], pacc[e], (float)(j - (ibase + rc)), ls, pv[e], dsv[e]);
      }
      if constexpr (HEAD_C1) {
#pragma unroll
        for (int e = 0; e < 16; ++e) dsv[e] *= sg.c1;
      }
      if (cls == TILE_PARTIAL) {
        // bit k: row ibase + k does not see key j
        const uint32_t hidden = ~key_bits(seen.lo - ibase, seen.hi - ibase);
        zero_hidden(pv, hidden);
        zero_hidden(dsv, hidden);
      }
      uint32_t pp[8], pd[8];
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        pp[w] = pack_bf16x2(pv[2 * w], pv[2 * w + 1]);
        pd[w] = pack_bf16x2(dsv[2 * w], dsv[2 * w + 1]);
      }
      // dV^T += dO^T P, dK^T += Q^T dS, 16-row chunk by chunk
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const int c = 2 * qb + half;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const char* qa = St + 16 * c * RP;
          const char* da = St + T_BYTES + 16 * c * RP;
          const int lo_off = t_lane ^ (64 * db), hi_off = t_lane8 ^ (64 * db);
          const i16x4_t qlo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(qa + lo_off));
          const i16x4_t qhi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(qa + hi_off));
          const i16x4_t dlo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(da + lo_off));
          const i16x4_t dhi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(da + hi_off));
          const bf16x8_t aq = __builtin_bit_cast(bf16x8_t, (i16x8_t)__builtin_shufflevector(qlo, qhi, 0, 1, 2, 3, 4, 5, 6, 7));
          const bf16x8_t ado = __builtin_bit_cast(bf16x8_t, (i16x8_t)__builtin_shufflevector(dlo, dhi, 0, 1, 2, 3, 4, 5, 6, 7));
          const u32x4_t wp = {pp[4 * half], pp[4 * half + 1], pp[4 * half + 2], pp[4 * half + 3]};
          const u32x4_t wd = {pd[4 * half], pd[4 * half + 1], pd[4 * half + 2], pd[4 * half + 3]};
          dv[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ado, __builtin_bit_cast(bf16x8_t, wp), dv[db], 0, 0, 0);
          dk[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(aq, __builtin_bit_cast(bf16x8_t, wd), dk[db], 0, 0, 0);
        }
      }
    }
  }

  if (okj) {
    uint16_t* kdst = dkh + (int64_t)j * dkrs + 4 * lh;
    uint16_t* vdst = dvh + (int64_t)j * dvrs + 4 * lh;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        u32x2_t wk, wv;
        wk[0] = pack_bf16x2(dk[db][4 * gq + 0] * c1u, dk[db][4 * gq + 1] * c1u);
        wk[1] = pack_bf16x2(dk[db][4 * gq + 2] * c1u, dk[db][4 * gq + 3] * c1u);
        wv[0] = pack_bf16x2(dv[db][4 * gq + 0], dv[db][4 * gq + 1]);
        wv[1] = pack_bf16x2(dv[db][4 * gq + 2], dv[db][4 * gq + 3]);
        *(u32x2_t*)(kdst + 32 * db + 8 * gq) = wk;
        *(u32x2_t*)(vdst + 32 * db + 8 * gq) = wv;
      }
  }
}

}  // namespace chia
