// attn_fp8_kernel.h -- gfx950 forward attention with FP8 (OCP e4m3 or e5m2) operands.
//
// Semantics: the forward of attn_fwd_kernel.h (mask, score modifiers,
// normalisers) for q, k, v stored as float8 e4m3 or e5m2 with per-tensor
// dequantisation factors (real value = stored value * descale); o is bf16.
// Both products run on v_mfma_scale_f32_32x32x64_f8f6f4 (unit block scales),
// twice the bf16 matrix rate:
//   S^T[key, query] = K Q^T   A = K rows (two ds_read_b128 per lane), B = Q
//                             rows in VGPRs; both operands put the same 32
//                             bytes of d in the same (lane half, byte) slots,
//                             which is all the contraction needs;
//   O^T[d, query] += V^T P^T  B = P^T: the lane's own 32 weights (lane =
//                             query, keys 8w + 4h + {0..3} in dword w, h the
//                             lane half), rounded to e4m3; A =
//                             V^T gathered from the row-major V tile with
//                             ds_read_b64_tr_b8 -- within a 16-lane group,
//                             lane j + 8p receives byte j of the 8-byte
//                             chunks read by lanes 2t + p (t = 0..7), so
//                             pointing lane 2t + p at key 16 wp + 4h + (t & 3)
//                             + 8 (t >> 2), columns d0 + 8p, hands lane j + 8p
//                             the four-key groups of dwords 2 wp, 2 wp + 1 of
//                             column d0 + 8p + j -- the keys of the B operand.
// The row sum adds the e4m3 weights that PV uses: decoded back to fp32 on the
// vector ALU (D = 128) or on the matrix core (D = 64).  Softmax weights are
// 2^(x - m + 4) with a running max m that moves (rescaling O and l) only when
// a tile's max exceeds it by more than 4 (log2): weights stay <= 2^8 < 448,
// the e4m3 maximum, and weights down to 2^-13 of the row max stay normal.
// Sigmoid weights are scaled by 2^8; ReLU weights are clamped to 448.  One workgroup = 4 wavefronts x 32 query rows; K and V tiles of 64 keys
// are DMA'd HBM -> LDS (16-byte chunks XOR-swizzled by row) in four stages at
// head dim 64 (three at 128) with one barrier per tile, as in the bf16 kernels.
#pragma once
#include "attn_bwd_kernel.h"  // attn_fwd_kernel.h and zero_hidden

namespace chia {

typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) i32x2_t lds_i32x2_t;

constexpr int kFp8E4M3 = 0;  // MFMA operand format codes (cbsz / blgp): OCP e4m3
constexpr int kFp8E5M2 = 1;  //   and OCP e5m2
constexpr float kFp8Max = 448.0f;
// Softmax weights are 2^(x - m + kFp8Pre) with a running max m that moves
// only when a tile's max exceeds it by more than kFp8Lazy: weights <= 2^8.
constexpr float kFp8Pre = 4.0f;
constexpr float kFp8Lazy = 4.0f;

struct Fp8Params {
  const uint8_t* q;
  const uint8_t* k;
  const uint8_t* v;
  uint16_t* o;
  int64_t q_sb, q_sh, q_ss;  // element (= byte) strides: batch, head, seq
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;  // bf16 element strides
  const float* head_scale;
  const float* alibi_slopes;
  MaskSpec mask;
  int32_t B, H, residues, n_blk, n_wg;
  UDiv div_blk, div_res, div_h, div_group;
  float qk_scale;   // scale * q_descale * k_descale
  float v_descale;
  float softcap, bias, post_scale;
  // Packed sequences (null: fixed length): sequence b is tokens cu_seqlens[b]
  // .. cu_seqlens[b + 1] - 1 (batch strides 0), mask.S the longest length;
  // seq_order[i] is the sequence of batch slot i (longest first).
  const int32_t* cu_seqlens;
  const int32_t* seq_order;
  // Longest-first launch order for causal rows (fixed length, B H residues a
  // multiple of 8): the (b, h, residue) slices per XCD, 0 otherwise; and its divider.
  int32_t rank_hx;
  UDiv div_hx;
};

// Swizzled 16-byte slot of chunk c of row r in an fp8 tile of D-byte rows.
template <int D>
__device__ __forceinline__ int fp8_slot(int r, int c) {
  return c ^ (r & (D / 16 - 1));
}

// One 64-row fp8 tile (row stride rs bytes, rows from `row`, clamped to
// S - 1) into LDS at dst with the swizzle above; wavefront w of 4 moves
// chunks [(n 4 + w) 64, +64) for n < NDMA.
template <int D>
__device__ __forceinline__ void fp8_dma_rows(const uint8_t* base, int64_t rs, int row, int S, char* dst, int wave,
                                             int lane) {
  constexpr int DQ = D / 16;
  constexpr int NDMA = 64 * DQ / 256;
  const uint8_t* src = base + (int64_t)row * rs;
#pragma unroll
  for (int n = 0; n < NDMA; ++n) {
    const int pos = (n * 4 + wave) * 64 + lane;
    const int r = pos / DQ, slot = pos % DQ;
    const int rr = imin32(r, S - 1 - row);
    dma16s(src, (uint32_t)((int64_t)rr * rs + 16 * fp8_slot<D>(r, slot)), lds_addr(dst + (n * 4 + wave) * 1024));
  }
}

// Two e4m3 weights into bytes (2 HI, 2 HI + 1) of `old` (round to nearest even).
template <bool HI>
__device__ __forceinline__ int pk_fp8(float a, float b, int old) {
  return __builtin_amdgcn_cvt_pk_fp8_f32(a, b, old, HI);
}

// FMT: the storage format of q, k and v (kFp8E4M3 or kFp8E5M2); the weights
// P are e4m3 in either case.
template <int D, int NORM, bool ALIBI, bool SOFTCAP, int FMT>
__global__ __launch_bounds__(256, 2) void attn_fwd_fp8_kernel(const Fp8Params p) {
  static_assert(FMT == kFp8E4M3 || FMT == kFp8E5M2, "q, k, v are e4m3 or e5m2");
  constexpr int NW = 4, BN = 64, KB = 2;
  constexpr int RP = D;                 // LDS row pitch (bytes)
  constexpr int T_BYTES = BN * RP;
  constexpr int STAGE_BYTES = 2 * T_BYTES;
  constexpr int NS = D == 64 ? 4 : 3;  // LDS stages (head dim 64: 32 KB, still four workgroups per CU)
  constexpr int KC = D / 64;            // 64-deep steps of the QK^T MFMA
  constexpr int DB = D / 32;            // 32-row d blocks of O^T
  constexpr int NDMA2 = 2 * (BN * (D / 16) / 256);  // DMA loads per tile per wavefront (K and V)
  __shared__ __attribute__((aligned(1024))) char lds[NS * STAGE_BYTES];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane & 31, lh = lane >> 5;

  // workgroup -> (b, h, residue, 128-row block), the blocks with the most keys
  // first.  Causal rows (rank_hx > 0): XCD x (workgroups x, x + 8, ...) serves
  // slices [x rank_hx, (x + 1) rank_hx) and walks them rank by rank, every
  // slice's last block, then every slice's second to last, ..., so the longest
  // blocks all start first and the shortest fill the end of the launch.
  // Otherwise each XCD gets a contiguous range of slices, longest block first
  // per slice; packed sequences go round-robin to the XCDs.
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
  const int dil = p.mask.dil;
  const int hk = udiv(h, p.div_group);
  const int64_t t0 = seq.tok0 + r;  // the residue's first token
  const uint8_t* qh = p.q + b * p.q_sb + h * p.q_sh + t0 * p.q_ss;
  const uint8_t* kh = p.k + b * p.k_sb + hk * p.k_sh + t0 * p.k_ss;
  const uint8_t* vh = p.v + b * p.v_sb + hk * p.v_sh + t0 * p.v_ss;
  uint16_t* oh = p.o + b * p.o_sb + h * p.o_sh + t0 * p.o_ss;
  const int64_t qrs = p.q_ss * dil, krs = p.k_ss * dil, vrs = p.v_ss * dil, ors = p.o_ss * dil;

  // per-head score constants: x = log2-domain score (softmax) or the score itself
  const float c1 = p.qk_scale * (p.head_scale ? p.head_scale[h] : 1.0f);
  const float sl = (ALIBI && p.alibi_slopes) ? p.alibi_slopes[h] * (float)dil : 0.0f;
  // ALiBi without softcap seeds the QK^T accumulator with (sl / c1)(j - i): the
  // MFMA returns the biased score over c1 and the normalisers take their plain form.
  constexpr bool kBiasInit = ALIBI && !SOFTCAP;
  // ALiBi softmax walks the key tiles from the last to the first: the bias grows
  // with the key index, so a row's max is set on its first tile and O is rarely
  // rescaled after it.
  constexpr bool kRev = ALIBI && NORM == NORM_SOFTMAX;
  const float bq = kBiasInit ? sl / c1 : 0.0f;

  // this wavefront's 32 rows: Q as the MFMA B operand (lane = row, 32 bytes of d per 64)
  const int row0 = blk * 128 + 32 * wave;
  const int i = row0 + lq;
  const bool ok = i < g.S;
  i32x8_t qf[KC];
  {
    const uint8_t* qs = qh + (int64_t)(ok ? i : 0) * qrs + 32 * lh;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      const i32x4_t lo = *(const i32x4_t*)(qs + 64 * kc);
      const i32x4_t hi = *(const i32x4_t*)(qs + 64 * kc + 16);
      qf[kc] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
  }

  const int wg_hi = imin32(blk * 128 + 127, g.S - 1);
  const TileRange tr = tile_range(g, blk * 128, wg_hi, BN);
  const int ntiles = tr.n_pre + tr.n2;
  const bool wvalid = row0 < g.S;
  const int ra = row0, rb = imin32(row0 + 31, g.S - 1);

  f32x16_t oacc[DB];
#pragma unroll
  for (int db = 0; db < DB; ++db)
#pragma unroll
    for (int e = 0; e < 16; ++e) oacc[db][e] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;
  // D = 64 softmax: the row sums come from the matrix core, as one more block
  // of O^T whose V^T rows are all ones (e4m3 1.0 = 0x38): every register of
  // lsum holds the sum of the lane's row's e4m3 weights.  One MFMA per tile
  // replaces 32 VALU adds per lane, and the kernels are VALU-bound.
  constexpr bool kMfmaSum = NORM == NORM_SOFTMAX && D == 64;
  f32x16_t lsum;
#pragma unroll
  for (int e = 0; e < 16; ++e) lsum[e] = 0.f;

  // LDS lane offsets.  K rows (A operand of S^T): row 32 kb + lq, chunks 4 kc + 2 lh (+1).
  // V^T (A operand of O^T) by transposed reads: lane q of 16-lane group G reads key
  // 16 wp + 4 hh + (t & 3) + 8 (t >> 2) (t = q / 2), columns 32 db + 16 (G & 1) + 8 (q & 1).
  const int grp = lane >> 4, q16 = lane & 15;
  const int t_src = q16 >> 1, p_src = q16 & 1, hh = grp >> 1;
  const int v_key = 4 * hh + (t_src & 3) + 8 * (t_src >> 2);  // + 16 wp

  // Scalar work per tile is kept small (it issues on the critical path with
  // four wavefronts per SIMD): the stage by a mask where NS is a power of two;
  // a tile's first key stepped by one tile from the previous one's, computed in
  // full only at a block's first tile and at the seam between its prefix and
  // band tiles (separately for the DMA, which runs NS - 1 tiles ahead, and the
  // compute); the K / V row base a 32 x 32 -> 64-bit product (keys are
  // non-negative, a row step is below 2^25 bytes); and on tiles inside the
  // sub-sequence the DMA's per-lane offsets fixed once.
  auto stage_of = [](int it) -> uint32_t {
    if constexpr ((NS & (NS - 1)) == 0) return (uint32_t)it & (NS - 1);
    else return (uint32_t)it % NS;
  };
  const int dkey = kRev ? -BN : BN;
  const int seam = kRev ? tr.n2 : tr.n_pre;
  auto tile_key = [&](int it) { return tile_at(tr, kRev ? ntiles - 1 - it : it) * BN; };
  const uint32_t krs_u = (uint32_t)krs, vrs_u = (uint32_t)vrs;
  constexpr int NDMA = BN * (D / 16) / 256;  // 1 KB loads per wavefront per tile (each of K, V)
  uint32_t k_off[NDMA], v_off[NDMA];
#pragma unroll
  for (int n = 0; n < NDMA; ++n) {
    const int pos = (n * 4 + wave) * 64 + lane;
    const int row = pos / (D / 16), slot = pos % (D / 16);
    k_off[n] = (uint32_t)row * krs_u + 16 * fp8_slot<D>(row, slot);
    v_off[n] = (uint32_t)row * vrs_u + 16 * fp8_slot<D>(row, slot);
  }
  auto issue = [&](int it, int jt0) {
    char* st = lds + stage_of(it) * STAGE_BYTES;
    if (jt0 + BN <= g.S) {
      const uint8_t* kt = kh + (uint64_t)(uint32_t)jt0 * krs_u;
      const uint8_t* vt = vh + (uint64_t)(uint32_t)jt0 * vrs_u;
#pragma unroll
      for (int n = 0; n < NDMA; ++n) {
        dma16s(kt, k_off[n], lds_addr(st + (n * 4 + wave) * 1024));
        dma16s(vt, v_off[n], lds_addr(st + T_BYTES + (n * 4 + wave) * 1024));
      }
    } else {
      fp8_dma_rows<D>(kh, krs, jt0, g.S, st, wave, lane);
      fp8_dma_rows<D>(vh, vrs, jt0, g.S, st + T_BYTES, wave, lane);
    }
  };
  int dma_next = 0, jt_dma = 0;
  for (; dma_next < NS - 1 && dma_next < ntiles; ++dma_next) {
    jt_dma = (dma_next == 0 || dma_next == seam) ? tile_key(dma_next) : jt_dma + dkey;
    issue(dma_next, jt_dma);
  }
  // the class of a tile against this wavefront's rows (mask.h)
  const KeyRanges<BN> kr(g, wvalid, ra, rb);
  int jt0 = 0;
  // Q in registers before the loop: otherwise the compiler's wait for these
  // loads sinks into the loop as vmcnt(0), which also drains the K/V tiles in
  // flight on every tile (the compiler does not count the DMA)
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) asm volatile("" : "+v"(qf[kc]));

  for (int it = 0; it < ntiles; ++it) {
    // this tile has landed; the loads of up to NS - 2 later tiles may stay in flight
    {
      const int inflight = dma_next - (it + 1);
      if (NS >= 4 && inflight >= 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * NDMA2) : "memory");
      else if (inflight >= 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(NDMA2) : "memory");
      else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (dma_next < ntiles) {
      jt_dma = (dma_next == seam) ? tile_key(dma_next) : jt_dma + dkey;
      issue(dma_next, jt_dma);
      ++dma_next;
    }
    const char* St = lds + stage_of(it) * STAGE_BYTES;
    jt0 = (it == 0 || it == seam) ? tile_key(it) : jt0 + dkey;
    const int cls = key_class(kr, jt0);
    if (cls == TILE_EMPTY) continue;

    // S^T for the tile's two 32-key blocks
    f32x16_t sacc[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      if constexpr (kBiasInit) {
        const float b0 = bq * (float)(jt0 + 32 * kb + 4 * lh - i);
#pragma unroll
        for (int e = 0; e < 16; ++e) sacc[kb][e] = __builtin_fmaf(bq, (float)(8 * (e >> 2) + (e & 3)), b0);
      } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) sacc[kb][e] = 0.f;
      }
      const int kr = 32 * kb + lq;
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) {
        const int c0 = 4 * kc + 2 * lh;
        const i32x4_t lo = *(const i32x4_t*)(St + kr * RP + 16 * fp8_slot<D>(kr, c0));
        const i32x4_t hi = *(const i32x4_t*)(St + kr * RP + 16 * fp8_slot<D>(kr, c0 + 1));
        const i32x8_t a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
        sacc[kb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, qf[kc], sacc[kb], FMT, FMT, 0,
                                                                  0x7f7f7f7f, 0, 0x7f7f7f7f);
      }
    }

    // scores -> weights (lane = query i; register e of block kb = key jt0 + 32 kb + 8 (e >> 2) + (e & 3) + 4 lh).
    // Without softcap (ALiBi is in the accumulator) the score's scale folds into
    // the weight's first operation.
    constexpr bool kPlain = !SOFTCAP;
    // x: the score in log2 units for softmax (osc = log2 e), in natural units otherwise.
    //   no softcap: x = osc (c1 s + sl (j - i)) = fma(s, c1 osc, fma(sl osc, rc, base_kb))
    //   softcap:    x = osc cap tanh(u / cap) = fma(r, -2 cap osc, cap osc), r = 1 / (1 + 2^(2 u log2e / cap))
    // with rc = 8 (e >> 2) + (e & 3) the register's key offset and base_kb the block's first (j - i).
    constexpr float osc = NORM == NORM_SOFTMAX ? kLog2e : 1.0f;
    float x[KB][16];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      if constexpr (kPlain) {
#pragma unroll
        for (int e = 0; e < 16; ++e) x[kb][e] = sacc[kb][e];
      } else {
        const float lk = SOFTCAP ? 2.0f * kLog2e / p.softcap : osc;  // units of the linear part
        const float kql = c1 * lk, ksl = sl * lk;
        const float base = ALIBI ? ksl * (float)(jt0 + 32 * kb + 4 * lh - i) : 0.0f;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const float rc = (float)(8 * (e >> 2) + (e & 3));
          const float lin = ALIBI ? __builtin_fmaf(sacc[kb][e], kql, __builtin_fmaf(ksl, rc, base)) : sacc[kb][e] * kql;
          if constexpr (SOFTCAP) {
            const float rr = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(lin));
            // softmax keeps r: the max is a min over r and the affine map folds into the exponent
            x[kb][e] = NORM == NORM_SOFTMAX ? rr : __builtin_fmaf(rr, -2.0f * p.softcap * osc, p.softcap * osc);
          } else {
            x[kb][e] = lin;
          }
        }
      }
    }
    uint32_t hidden[KB] = {0u, 0u};
    if (cls == TILE_PARTIAL) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) hidden[kb] = hidden_bits(g, i, jt0 + 32 * kb + 4 * lh);
    }
    float pw[KB][16];
    if constexpr (NORM == NORM_SOFTMAX) {
      // working units: raw scores (plain, scaled by kq = c1 log2 e in the exponent) or log2 units
      const float kq = c1 * kLog2e;
      // softcap: x holds r, and the score is cA r + cB (cA < 0)
      const float cA = -2.0f * p.softcap * kLog2e, cB = p.softcap * kLog2e;
      if (cls == TILE_PARTIAL) {
        // hidden keys -> -inf (r: +inf): all ones where hidden (v_bfe_i32), then one bitwise blend
        uint32_t ninf;
        asm("s_mov_b32 %0, %1" : "=s"(ninf) : "i"(SOFTCAP ? 0x7f800000 : 0xff800000));
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            uint32_t m = (uint32_t)__builtin_amdgcn_sbfe((int)hidden[kb], 8 * (e >> 2) + (e & 3), 1);
            asm("" : "+v"(m));
            x[kb][e] = __uint_as_float((m & ninf) | (~m & __float_as_uint(x[kb][e])));
          }
      }
      float mx;
      if constexpr (SOFTCAP) {
        float mr = INFINITY;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int e = 0; e < 16; ++e) mr = fminf(mr, x[kb][e]);
        mr = -xhalf_max(-mr);
        mx = mr == INFINITY ? -INFINITY : __builtin_fmaf(mr, cA, cB);
      } else {
        mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int e = 0; e < 16; ++e) mx = fmaxf(mx, x[kb][e]);
        mx = xhalf_max(mx);
      }
      const float ml2 = kPlain ? mx * kq : mx;  // kq > 0 keeps the order; -inf stays -inf
      const float m_new = ml2 > m_run + kFp8Lazy ? ml2 : m_run;
      if (__any(m_new != m_run)) {
        const float alpha = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
        l_run *= alpha;
        if constexpr (kMfmaSum)
#pragma unroll
          for (int e = 0; e < 16; ++e) lsum[e] *= alpha;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int e = 0; e < 16; ++e) oacc[db][e] *= alpha;
        m_run = m_new;
      }
      const float m_use = (m_run == -INFINITY) ? 0.f : m_run - kFp8Pre;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          float arg;
          if constexpr (kPlain) arg = __builtin_fmaf(x[kb][e], kq, -m_use);
          else if constexpr (SOFTCAP) arg = __builtin_fmaf(x[kb][e], cA, cB - m_use);
          else arg = x[kb][e] - m_use;
          pw[kb][e] = __builtin_amdgcn_exp2f(arg);
        }
    } else {
      // sigmoid: 2^8 / (1 + 2^(-(t + bias) log2 e)) = rcp(2^-8 e + 2^-8); ReLU: clamp(t, 0, 448)
      const float nk = kPlain ? -c1 * kLog2e : -kLog2e, nb = -p.bias * kLog2e;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          float w;
          if constexpr (NORM == NORM_SIGMOID) {
            const float ex = __builtin_amdgcn_exp2f(__builtin_fmaf(x[kb][e], nk, nb));
            w = __builtin_amdgcn_rcpf(__builtin_fmaf(ex, 1.0f / 256.0f, 1.0f / 256.0f));
          } else {
            const float t = kPlain ? x[kb][e] * c1 : x[kb][e];
            w = __builtin_amdgcn_fmed3f(t, 0.0f, kFp8Max);
          }
          pw[kb][e] = w;
        }
        if (cls == TILE_PARTIAL) zero_hidden(pw[kb], hidden[kb]);
      }
    }

    // P^T as the B operand: dword w = 4 kb + (e >> 2) holds keys 8 w + 4 lh + (e & 3)
    i32x8_t pb;
#pragma unroll
    for (int w = 0; w < 8; ++w) {
      const int kb = w >> 2, e0 = 4 * (w & 3);
      int d = pk_fp8<false>(pw[kb][e0], pw[kb][e0 + 1], 0);
      d = pk_fp8<true>(pw[kb][e0 + 2], pw[kb][e0 + 3], d);
      pb[w] = d;
    }
    // D = 128 softmax: the row sum adds the e4m3 weights that PV uses, decoded
    // from pb, so the rounding of a row's dominant weight cancels in o = PV / l
    // (with the lazy max that weight is rarely a power of two; summing the fp32
    // weights instead left up to 2^-4 of it in the numerator alone)
    if constexpr (NORM == NORM_SOFTMAX && !kMfmaSum) {
      float ls = 0.f;
#pragma unroll
      for (int w = 0; w < 8; ++w) {
        const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(pb[w], false);
        const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(pb[w], true);
        ls += (lo[0] + lo[1]) + (hi[0] + hi[1]);
      }
      l_run += ls;
    }

    // O^T += V^T P^T, one MFMA per 32-row d block
    const char* Vt = St + T_BYTES;
#pragma unroll
    for (int db = 0; db < DB; ++db) {
      const int chunk = 2 * db + (grp & 1);
      i32x2_t t2[4];
#pragma unroll
      for (int wp = 0; wp < 4; ++wp) {
        const int key = 16 * wp + v_key;
        const char* src = Vt + key * RP + 16 * fp8_slot<D>(key, chunk) + 8 * p_src;
        t2[wp] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2_t*)src);
      }
      const i32x8_t va = __builtin_shufflevector(__builtin_shufflevector(t2[0], t2[1], 0, 1, 2, 3),
                                                 __builtin_shufflevector(t2[2], t2[3], 0, 1, 2, 3), 0, 1, 2, 3, 4, 5,
                                                 6, 7);
      oacc[db] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(va, pb, oacc[db], FMT, kFp8E4M3, 0, 0x7f7f7f7f,
                                                                 0, 0x7f7f7f7f);
    }
    if constexpr (kMfmaSum) {
      const i32x8_t ones = {0x38383838, 0x38383838, 0x38383838, 0x38383838,
                            0x38383838, 0x38383838, 0x38383838, 0x38383838};
      lsum = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ones, pb, lsum, kFp8E4M3, kFp8E4M3, 0, 0x7f7f7f7f, 0,
                                                             0x7f7f7f7f);
    }
  }

  // epilogue: o = O^T^T * v_descale / (2^8 l) (softmax) or * v_descale * post / 2^8
  if (ok) {
    float f;
    if constexpr (NORM == NORM_SOFTMAX) {
      const float lt = kMfmaSum ? lsum[0] : xhalf_sum(l_run);
      f = lt > 0.f ? p.v_descale / lt : 0.f;
    } else if constexpr (NORM == NORM_SIGMOID) {
      f = p.v_descale * p.post_scale * (1.0f / 256.0f);
    } else {
      f = p.v_descale * p.post_scale;
    }
    uint16_t* dst = oh + (int64_t)i * ors + 4 * lh;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        u32x2_t w;
        w[0] = pack_bf16x2(oacc[db][4 * gq + 0] * f, oacc[db][4 * gq + 1] * f);
        w[1] = pack_bf16x2(oacc[db][4 * gq + 2] * f, oacc[db][4 * gq + 3] * f);
        *(u32x2_t*)(dst + 32 * db + 8 * gq) = w;
      }
  }  // (lanes l and l + 32 hold the same row, so the half-wave sum above runs on both or neither)
}

using Fp8KernelFn = void (*)(Fp8Params);

}  // namespace chia
