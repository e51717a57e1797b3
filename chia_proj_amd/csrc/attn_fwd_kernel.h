// attn_fwd_kernel.h -- the gfx950 forward-attention core behind every variant.
//
// Reference semantics: the eager closures of extra_bench.py:32-62 (score
// s = q k^T * scale, score modifier, mask, normaliser in fp32, p rounded to
// bf16, p @ v) and sigmoid_fix.py:34-40 (sigmoid first, then zero the masked
// entries).  This is an original CDNA4 design, not a port of the reference's
// Triton kernels.
//
// Work decomposition
//   * one workgroup = NW wavefronts and a PAIR of row blocks (32 NW rows each)
//     of one (batch, head, dilation residue); each wavefront owns 32 rows of
//     each block (its two "query blocks" qb = 0, 1).  For causal masks without
//     a window the pair is (i, n-1-i): every workgroup then does the same
//     amount of work whatever the dispatcher's placement, which a contiguous
//     split cannot give when all workgroups are resident at once.  Otherwise
//     the pair is (2i, 2i+1);
//   * the KV loop walks only the key tiles (BN = 64 keys) the mask can reach
//     (prefix tiles + the band hull).  K and V tiles go from HBM straight into
//     LDS with global_load_lds_dwordx4 (no VGPR staging) into four stages
//     (two for 2-wavefront workgroups), up to three tiles ahead of the one
//     computed, one barrier per step.
//     Each wavefront classifies the tile against its own rows and skips it
//     (EMPTY), runs it unmasked (FULL) or with the per-element predicate
//     (PARTIAL); band tiles inside precomputed ranges (fast_ranges) are known
//     to be FULL without classifying;
//   * a tile is one step: four 32 x 32 score blocks (two query blocks x two
//     key blocks, PAIR) or, when only block 1 sees it, two blocks of block 1
//     (WIDE); two consecutive tiles that only block 1 sees, in every
//     wavefront, make one four-block step (WIDE2).  All QK^T MFMAs of a step
//     come before its softmax.
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
//   LDS tiles are dense rows of 2D bytes whose 16-byte chunks are XOR-swizzled
//   (a DMA load fills 1 KB contiguously, so rows cannot be padded): K chunk c
//   of row r sits in slot k_slot(r, c), so the 16 rows of a ds_read_b128 pass
//   hit distinct bank groups; V chunk c sits in slot v_slot(r, c), so the
//   four rows x 64 bytes of one 32-lane transposed-read pass do.  With rows
//   of a multiple of 128 bytes every fragment offset is a per-lane base XOR a
//   compile-time constant.
//   The softmax runs per tile in the exp2 domain against a lazily moved
//   reference max.  A tile's weights are first computed against the running
//   reference m; only when a row has no reference yet, or a lane's partial
//   row sum over the tile exceeds kLazyBound (some weight may exceed it), is
//   the tile's row max computed: the reference then moves to it when it
//   exceeds m by more than kRescaleLog2 (rescaling O and l), and the tile's
//   weights are recomputed.  So p <= kLazyBound, and the row max -- about a
//   quarter of the plain softmax's vector instructions per score -- is skipped
//   on almost every tile.  ALiBi's bias grows with the key index, so its
//   kernels walk the key tiles from the last to the first: a row's first tile
//   then sets the reference, and the later tiles, lower by the slope times
//   their distance, stay under it.
//   The row sum l accumulates the bf16-rounded weights the PV MFMA consumes
//   (v_dot2c_f32_bf16 against (1, 1): one instruction per two weights).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lds_layout.h"
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
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kRescaleLog2 = 8.0f;  // lazy-rescale threshold (log2 units)
constexpr float kLazyBound = 65536.0f;  // partial row sum of one tile that triggers an exact max
constexpr int kBN = 64;

// KeyRanges<N>::classify (mask.h) as scalar compares and selects, for a key
// offset the wavefront shares: ten scalar instructions, no branch.  The
// compiler's form of the same tests combines 64-bit condition masks, about
// twice the instructions, in a loop where scalar issue is on the critical path.
template <int N>
__device__ __forceinline__ int key_class(const KeyRanges<N>& kr, int c) {
  static_assert(TILE_EMPTY == 0 && TILE_FULL == 1 && TILE_PARTIAL == 2, "class codes");
  int cls, t;
  asm("s_sub_u32 %1, %2, %5\n\t"
      "s_cmp_le_u32 %1, %6\n\t"
      "s_cselect_b32 %0, 2, 0\n\t"   // some key in the hull: PARTIAL
      "s_cmp_lt_i32 %2, %7\n\t"
      "s_cselect_b32 %0, 2, %0\n\t"  // the first key in the prefix: PARTIAL
      "s_sub_u32 %1, %2, %3\n\t"
      "s_cmp_le_u32 %1, %4\n\t"
      "s_cselect_b32 %0, 1, %0\n\t"  // every key in the common interval: FULL
      "s_cmp_le_i32 %2, %8\n\t"
      "s_cselect_b32 %0, 1, %0"      // every key in the prefix: FULL
      : "=&s"(cls), "=&s"(t)
      : "s"(c), "s"(kr.bf_lo), "s"(kr.bf_span), "s"(kr.v_lo), "s"(kr.v_span), "s"(kr.pfx), "s"(kr.pf_hi)
      : "scc");
  return cls;
}

// RowRanges<M>::classify (mask.h) the same way, for a row tile start the
// wavefront shares: twelve scalar instructions, no branch.
template <int M>
__device__ __forceinline__ int row_class(const RowRanges<M>& rr, int a) {
  int cls, b, t, u;
  asm("s_add_i32 %1, %4, %9\n\t"   // b = min(a + M - 1, S - 1)
      "s_min_i32 %1, %1, %5\n\t"
      "s_sub_i32 %2, %1, %6\n\t"
      "s_sub_i32 %3, %7, %4\n\t"
      "s_min_i32 %2, %2, %3\n\t"
      "s_cmp_ge_i32 %2, 0\n\t"
      "s_cselect_b32 %0, 2, 0\n\t"   // b >= v_lo and a <= v_hi: PARTIAL
      "s_sub_i32 %2, %4, %8\n\t"
      "s_sub_i32 %3, %10, %1\n\t"
      "s_min_i32 %2, %2, %3\n\t"
      "s_cmp_ge_i32 %2, 0\n\t"
      "s_cselect_b32 %0, 1, %0"      // a >= f_lo and b <= f_hi: FULL
      : "=&s"(cls), "=&s"(b), "=&s"(t), "=&s"(u)
      : "s"(a), "s"(rr.last), "s"(rr.v_lo), "s"(rr.v_hi), "s"(rr.f_lo), "n"(M - 1), "s"(rr.f_hi)
      : "scc");
  return cls;
}

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
  int32_t n_pairs;            // row-block pairs per (b, h, residue 0)
  int32_t zigzag;             // pair blocks (i, n-1-i) instead of (2i, 2i+1)
  int32_t n_wg;
  UDiv div_pairs, div_res, div_h;  // dividers by n_pairs, residues, H
  UDiv div_group;                  // by query heads per K/V head (GQA / MQA)
  float* lse;                      // softmax: fp32 log-sum-exp of the scores, or nullptr
  int64_t lse_sb, lse_sh, lse_ss;  // its strides: batch, head, token
  const int32_t* cu_seqlens;       // packed sequences: [B + 1] token offsets, or nullptr
  const int32_t* seq_order;        // packed sequences: dispatch order of the B sequences, or nullptr
  float scale, softcap, bias, post_scale;
  // Longest-first launch order (rows whose work grows with the block index;
  // fixed length, B H residues a multiple of 8): the (b, h, residue) slices
  // per XCD, 0 otherwise; and its divider.  See rank_order().
  int32_t rank_hx;
  UDiv div_hx;
};

// Workgroup -> (slice, unit) in the longest-first order: XCD x (workgroups x,
// x + 8, ...) serves slices [x hx, (x + 1) hx) and walks them rank by rank,
// every slice's last unit, then every slice's second to last, ..., so the
// units with the most keys all start first and the shortest fill the end of
// the launch.  Bijective when the launch has 8 hx n_units workgroups.
struct SliceUnit {
  int slice, unit;
};
__device__ __forceinline__ SliceUnit rank_order(int x, int hx, UDiv div_hx, int n_units) {
  const int xcd = x & 7, local = x >> 3;
  const int rank = udiv(local, div_hx);
  return SliceUnit{xcd * hx + (local - rank * hx), n_units - 1 - rank};
}

// Packed sequences: sequence b's first token and length (at most the launch's
// S); fixed-length batches: 0 and S.
struct SeqSpan {
  int64_t tok0;
  int32_t len;
};
// Packed sequences: the launch's i-th sequence slot runs sequence seq_order[i].
__device__ __forceinline__ int seq_of(const int32_t* seq_order, int i) { return seq_order ? seq_order[i] : i; }

__device__ __forceinline__ SeqSpan seq_span(const int32_t* cu_seqlens, int b, int32_t S) {
  SeqSpan s{0, S};
  if (cu_seqlens) {
    const int32_t t0 = cu_seqlens[b];
    s.tok0 = t0;
    s.len = imax32(imin32(cu_seqlens[b + 1] - t0, S), 0);
  }
  return s;
}

// Waves per SIMD the register budget targets: two at head_dim 64 (the
// hardware then overlaps one wave's softmax with the other's MFMAs), one at
// head_dim 128 (its O accumulator alone is 128 VGPRs).
template <int D>
struct Occupancy {
  static constexpr int value = D == 64 ? 2 : 1;
};

typedef __attribute__((address_space(3))) void lds_void_t;

template <bool V>
struct BoolTag {
  static constexpr bool value = V;
};
template <int V>
struct IntTag {
  static constexpr int value = V;
};

// The software-pipelined run (below) is compiled where its registers fit
// without spilling: 4 wavefronts, sigmoid / ReLU without a score modifier.
template <int D, int NW, int NORM, bool ALIBI, bool SOFTCAP>
struct Pipelined {
  static constexpr bool value = NW == 4 && NORM != NORM_SOFTMAX && !ALIBI && !SOFTCAP;
};

// 32-bit LDS address of a generic pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
}

// One 16-byte-per-lane HBM -> LDS DMA load from sbase + voff (uniform base,
// per-lane byte offset): lane l's chunk lands at lds_base + 16 l.  Issued through asm so that the compiler does not track it:
// it would otherwise treat every later LDS read as aliasing the transfer and
// wait for all loads in flight.  The kernel orders the transfers itself with
// explicit vmcnt waits and barriers.
// The base is made explicitly wave-uniform (it is by construction) so that
// it always lands in scalar registers.  readfirstlane returns int: each half
// goes back through uint32_t so that the low word is not sign-extended.
__device__ __forceinline__ void dma16s(const void* sbase, uint32_t voff, uint32_t lds_base) {
  const uint64_t v = (uint64_t)(uintptr_t)sbase;
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
  const uint64_t u = ((uint64_t)hi << 32) | (uint64_t)lo;
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(u), "{m0}"(lds_base) : "memory");
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

// max(x, 0) as one v_max_i32 on the bit pattern: negative floats and -0 are
// negative integers, non-negative floats keep their order as integers.
// (fmaxf of an MFMA result costs a second v_max that first quiets a possible
// signalling NaN; here a NaN of positive sign propagates, as torch.relu does.)
__device__ __forceinline__ float relu0(float x) {
  const int i = __builtin_bit_cast(int, x);
  return __builtin_bit_cast(float, i > 0 ? i : 0);
}

template <int D, int NW, int NORM, bool ALIBI, bool SOFTCAP>
__global__ __launch_bounds__(NW * 64, Occupancy<D>::value) void attn_fwd_kernel(const FwdParams p) {
  constexpr int BN = kBN;
  constexpr int NT = NW * 64;        // threads per workgroup
  constexpr int QB = 2;              // 32-row query blocks per wavefront (one per row block)
  constexpr int BMH = NW * 32;       // rows per row block
  constexpr int KB = BN / 32;        // 32-key blocks per tile
  constexpr int DK = D / 16;         // k-steps of the QK^T MFMA
  constexpr int DB = D / 32;         // 32-row d blocks of O^T
  constexpr int DQ = D / 8;          // 16-byte chunks per K/V row
  constexpr int RP = 2 * D;          // LDS row pitch (bytes)
  constexpr int NDMA = BN * DQ / NT; // 1 KB DMA loads per wavefront per tile (each of K, V)
  constexpr int K_BYTES = BN * RP;
  constexpr int STAGE_BYTES = 2 * K_BYTES;  // K tile + V tile
  static_assert(NDMA >= 1 && BN * DQ % NT == 0, "tile does not split into whole DMA loads");
  static_assert(RP % 128 == 0, "rows must be whole multiples of 128 bytes for the XOR offsets");
  static_assert(KB == 2, "a WIDE step covers the two key blocks of a tile");
  constexpr bool kPlainSoftmax = (NORM == NORM_SOFTMAX) && !ALIBI && !SOFTCAP;
  // ALiBi without softcap: the bias enters the QK^T accumulator as its initial
  // value, (sl / c1)(j - i) (c1 > 0), so the MFMA returns (biased score) / c1
  // and the normaliser takes its unbiased form -- one VALU per score fewer than
  // adding the bias afterwards.  Softmax then runs the plain exponent.
  constexpr bool kBiasInit = ALIBI && !SOFTCAP;
  constexpr bool kScaledSoftmax = kPlainSoftmax || (kBiasInit && NORM == NORM_SOFTMAX);  // exponent fma(s, kq, -m)
  constexpr bool kBiasFold = kBiasInit && NORM == NORM_SOFTMAX;  // the block bias in the exponent (below)
  constexpr bool kRawRelu = (NORM == NORM_RELU) && !ALIBI && !SOFTCAP;
  // Softcapped softmax keeps r = 1 / (1 + 2^(2 s log2e / cap)) per score; the
  // capped score in log2 units is t = sc_a r + sc_b (sc_a < 0), folded into
  // the exponential's argument together with the reference max.
  constexpr bool kCapR = SOFTCAP && NORM == NORM_SOFTMAX;
  constexpr bool kSigFold = NORM == NORM_SIGMOID && !ALIBI && !SOFTCAP;
  // ALiBi softmax walks its key tiles from the last to the first: the bias
  // grows with the key index, so a row's first tile fixes its max and the
  // later ones stay under it, as the tile max only on demand needs.
  constexpr bool kRev = ALIBI && NORM == NORM_SOFTMAX;
  constexpr bool kLazyMax = !ALIBI || kRev;  // softmax: the tile max only on demand

  constexpr bool kPipe = Pipelined<D, NW, NORM, ALIBI, SOFTCAP>::value;
  // LDS stages: 4 for 4-wavefront workgroups (up to three tiles in flight;
  // WIDE2 steps hold two), 2 for 2-wavefront ones.
  constexpr int NS = NW == 4 ? 4 : 2;
  static_assert((NS & (NS - 1)) == 0, "stage index is a mask");
  constexpr bool kWide2 = NW == 4 && !kPipe;  // (the pipelined kernels keep their registers for the run)
  __shared__ __attribute__((aligned(1024))) char lds[NS * STAGE_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane & 31, lh = lane >> 5;

  // ---- workgroup -> (batch, head, residue, row-block pair) -----------------
  // Packed sequences of unequal length: consecutive workgroups go round-robin
  // to the XCDs so every XCD gets a share of every sequence's work.
  int bhr, pr;
  if (p.rank_hx > 0) {
    const SliceUnit su = rank_order((int)blockIdx.x, p.rank_hx, p.div_hx, p.n_pairs);
    bhr = su.slice;
    pr = su.unit;
  } else {
    const int L = p.cu_seqlens ? (int)blockIdx.x : xcd_remap(blockIdx.x, p.n_wg);
    bhr = udiv(L, p.div_pairs);
    pr = L - bhr * p.n_pairs;
  }
  const int bh = udiv(bhr, p.div_res);
  const int r = bhr - bh * p.residues;
  const int bs = udiv(bh, p.div_h);
  const int h = bh - bs * p.H;
  const int b = seq_of(p.seq_order, bs);
  const SeqSpan seq = seq_span(p.cu_seqlens, b, p.mask.S);
  MaskSpec ms = p.mask;
  ms.S = seq.len;
  const MaskGeom g = residue_geom(ms, r);
  const int nblk = (g.S + BMH - 1) / BMH;  // row blocks of this residue
  int blk0, blk1;
  if (p.zigzag) {
    blk0 = pr;
    blk1 = nblk - 1 - pr;
    if (blk1 < blk0) return;  // whole workgroup, before any barrier
    if (blk1 == blk0) blk1 = -1;
  } else {
    blk0 = 2 * pr;
    blk1 = 2 * pr + 1;
    if (blk0 >= nblk) return;
    if (blk1 >= nblk) blk1 = -1;
  }

  const int dil = p.mask.dil;
  const int64_t t0 = seq.tok0 + r;  // the residue's first token
  const uint16_t* qh = p.q + b * p.q_sb + h * p.q_sh + t0 * p.q_ss;
  const int hk = udiv(h, p.div_group);  // K/V head of query head h
  const uint16_t* kh = p.k + b * p.k_sb + hk * p.k_sh + t0 * p.k_ss;
  const uint16_t* vh = p.v + b * p.v_sb + hk * p.v_sh + t0 * p.v_ss;
  uint16_t* oh = p.o + b * p.o_sb + h * p.o_sh + t0 * p.o_ss;
  const int64_t qrs = p.q_ss * dil, krs = p.k_ss * dil, vrs = p.v_ss * dil, ors = p.o_ss * dil;

  // ---- per-head score constants --------------------------------------------
  const float hs = p.head_scale ? p.head_scale[h] : 1.0f;
  const float slope = ALIBI && p.alibi_slopes ? p.alibi_slopes[h] : 0.0f;  // null: zero slopes
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
  const float bq = kBiasInit ? sl / c1 : 0.f;  // ALiBi bias per key step, in units of q . k
  // ALiBi softmax: S starts from bq rc(e), the bias of register e's key
  // offset rc(e) inside a 32-key block (the same registers for every block),
  // and the rest, bq (j0 - i) for the block's first key j0 and the lane's row
  // i, joins the exponent as one constant per block.  (ALiBi sigmoid / ReLU
  // seed S with the whole bias: their kernels have no registers to spare.)
  f32x16_t bias_rc;
#pragma unroll
  for (int e = 0; e < 16; ++e) bias_rc[e] = kBiasFold ? bq * (float)(8 * (e >> 2) + (e & 3)) : 0.f;
  // Plain sigmoid: Q is pre-scaled by kq (one bf16 rounding per element, at
  // load), so a score is already the exponent, and the bias enters as the
  // factor 2^k0: p = 1 / (1 + 2^k0 2^s).  The host routes a bias whose 2^k0
  // is not a normal float to the general path (ALIBI with null slopes).
  const float sig_c =
      kSigFold ? __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(__builtin_amdgcn_exp2f(k0)))) : 0.f;

  // ---- wavefront rows, Q fragments, per-row key intervals -------------------
  int row0[QB];      // first row of this wavefront's 32-row query block qb
  bool valid[QB];
  row0[0] = blk0 * BMH + 32 * wave;
  row0[1] = (blk1 >= 0 ? blk1 : blk0) * BMH + 32 * wave;
  valid[0] = row0[0] < g.S;
  valid[1] = blk1 >= 0 && row0[1] < g.S;

  bf16x8_t qf[QB][DK];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int i = row0[qb] + lq;
    const bool ok = valid[qb] && i < g.S;
    const uint16_t* src = qh + (int64_t)(ok ? i : 0) * qrs + 8 * lh;
#pragma unroll
    for (int kk = 0; kk < DK; ++kk) {
      u32x4_t val = *(const u32x4_t*)(src + 16 * kk);
      if (!ok) val = u32x4_t{0u, 0u, 0u, 0u};
      if constexpr (kSigFold) {
#pragma unroll
        for (int w = 0; w < 4; ++w)
          val[w] = pack_bf16x2(__uint_as_float(val[w] << 16) * kq, __uint_as_float(val[w] & 0xffff0000u) * kq);
      }
      qf[qb][kk] = __builtin_bit_cast(bf16x8_t, val);
    }
  }

  // ---- key intervals of every wavefront's blocks, evaluated in lanes ---------
  // Lane l works for wavefront w = l % NW: the interval ends key_lo / key_hi
  // at the first (a) and last (b) row of w's two query blocks, and w's fast
  // ranges.  A wavefront reads its own values from lane `wave`, and the
  // workgroup's tile range and WIDE2 range from lanes 0..NW-1, so this set-up
  // runs as a handful of vector instructions instead of some thousand scalar
  // ones (the scalar unit is shared by every wavefront of the CU).
  int lk[QB][4];  // key_lo(a), key_hi(b), key_lo(b), key_hi(a)
  FastRanges lf;
  {
    const int lw = lane & (NW - 1);
    int la[QB];
    bool lv[QB];
    la[0] = blk0 * BMH + 32 * lw;
    la[1] = (blk1 >= 0 ? blk1 : blk0) * BMH + 32 * lw;
    lv[0] = la[0] < g.S;
    lv[1] = blk1 >= 0 && la[1] < g.S;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int lb = imin32(la[qb] + 31, g.S - 1);
      lk[qb][0] = key_lo(g, la[qb]);
      lk[qb][1] = key_hi(g, lb);
      lk[qb][2] = key_lo(g, lb);
      lk[qb][3] = key_hi(g, la[qb]);
    }
    lf = fast_ranges_keys(g.S, lk[0][2], lk[0][3], lk[0][0], lk[0][1], lv[0], lk[1][2], lk[1][3], lv[1], BN);
  }

  // ---- KV tiles this workgroup visits ---------------------------------------
  // hull of the workgroup's rows: from the first row of wavefront 0's block 0
  // to the last row of wavefront NW-1's block 1 (block 0 when there is none)
  const TileRange tr =
      tile_range_keys(g, __builtin_amdgcn_readlane(lk[0][0], 0), __builtin_amdgcn_readlane(lk[1][1], NW - 1), BN);
  const int ntiles = tr.n_pre + tr.n2;
  // the tile of step k, and whether it lies in the band (not the prefix)
  auto seq_tile = [&](int k) __attribute__((always_inline)) { return tile_at(tr, kRev ? ntiles - 1 - k : k); };
  auto in_band = [&](int k) __attribute__((always_inline)) { return kRev ? k < tr.n2 : k >= tr.n_pre; };

  // Global -> LDS DMA.  Load n of wavefront w fills LDS chunks
  // [(n NW + w) 64, +64) of the K (or V) tile: lane l moves the 16-byte chunk
  // that belongs in slot (pos % DQ) of row pos / DQ, i.e. logical chunk
  // slot ^ swizzle(row).  The per-lane byte offsets from the tile's first row
  // are fixed; a tile adds its (uniform) row base.  Rows past the end re-read
  // the last row (finite values; the mask gives their scores p = 0).
  uint32_t k_dma[NDMA], v_dma[NDMA];
#pragma unroll
  for (int n = 0; n < NDMA; ++n) {
    const int pos = (n * NW + wave) * 64 + lane;
    const int row = pos / DQ, slot = pos % DQ;
    k_dma[n] = (uint32_t)(2 * ((int64_t)row * krs + 8 * k_slot<D>(row, slot)));
    v_dma[n] = (uint32_t)(2 * ((int64_t)row * vrs + 8 * v_slot<D>(row, slot)));
  }
  auto issue_tile = [&](int jt0, int stage) {
    char* kst = lds + stage * STAGE_BYTES;
    const uint16_t* kt = kh + (int64_t)jt0 * krs;
    const uint16_t* vt = vh + (int64_t)jt0 * vrs;
    if (jt0 + BN <= g.S) {
#pragma unroll
      for (int n = 0; n < NDMA; ++n) {
        const uint32_t lbase = lds_addr(kst + (n * NW + wave) * 1024);
        dma16s(kt, k_dma[n], lbase);
        dma16s(vt, v_dma[n], lbase + K_BYTES);
      }
    } else {
#pragma unroll
      for (int n = 0; n < NDMA; ++n) {
        const int pos = (n * NW + wave) * 64 + lane;
        const int row = pos / DQ, slot = pos % DQ;
        const int rr = imin32(row, g.S - 1 - jt0);
        const uint32_t lbase = lds_addr(kst + (n * NW + wave) * 1024);
        dma16s(kt, (uint32_t)(2 * ((int64_t)rr * krs + 8 * k_slot<D>(row, slot))), lbase);
        dma16s(vt, (uint32_t)(2 * ((int64_t)rr * vrs + 8 * v_slot<D>(row, slot))), lbase + K_BYTES);
      }
    }
  };

  // ---- DMA schedule: NS LDS stages, one barrier per step --------------------
  // Tiles [0, dma_next) have been issued; tile T goes to stage T % NS.  A
  // step over tiles [it, it + n) waits until those have landed (the loads of
  // later tiles stay in flight), then the barrier makes every wavefront's
  // part of them visible, and the DMA continues up to tile oldest + NS - 1,
  // where `oldest` is the first tile still read after this barrier: the tile
  // it overwrites, oldest - 1, was last read before it.  (oldest = it, or
  // it - 1 in kernels with a pipelined run, which reads the pending step's V
  // tile after the next tile's barrier.)  Every wavefront loads part of every
  // tile, so the steps, barriers and DMA issues must be the same in all
  // wavefronts of the workgroup: only workgroup-uniform values decide them
  // (the tile range, the WIDE2 range below, and `oldest` fixed per kernel,
  // since the other wavefronts may still be inside their pipelined run).
  // The barrier is a bare s_barrier: a __syncthreads() fence would also wait
  // for the loads still in flight.
  // A step frees as many stages as it had tiles, so a sync issues at most
  // kIssue tiles (the previous step's count), and at most kFly tiles beyond
  // the step's own are in flight when it waits: NS - 2, or NS - 3 where the
  // pipelined run keeps one more stage.  Waiting for fewer tiles in flight
  // than there are is always safe, so the vmcnt cases stop at kFly.
  constexpr int kIssue = kWide2 ? 2 : 1;
  constexpr int kFly = NS - (kPipe ? 3 : 2);
  static_assert(kFly >= 0 && kFly <= 2, "vmcnt cases cover up to two tiles in flight");
  int dma_next = 0;
  auto issue_upto = [&](int last) __attribute__((always_inline)) {
    last = imin32(last, ntiles - 1);
#pragma unroll
    for (int k = 0; k < kIssue; ++k)
      if (dma_next <= last) {
        issue_tile(seq_tile(dma_next) * BN, dma_next & (NS - 1));
        ++dma_next;
      }
  };
  auto sync_step = [&](int it, int n, int oldest) __attribute__((always_inline)) {
    const int inflight = dma_next - (it + n);  // tiles allowed to stay in flight
    if (kFly >= 2 && inflight >= 2) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * NDMA) : "memory");
    else if (kFly >= 1 && inflight >= 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * NDMA) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    issue_upto(oldest + NS - 1);
  };
  auto sync_tile = [&](int it) __attribute__((always_inline)) { sync_step(it, 1, kPipe ? it - 1 : it); };
  // prologue: the first kFly + 1 tiles (the first sync issues the next one),
  // issued before the per-block set-up below so the loads overlap it
  for (int t = 0; t <= kFly && t < ntiles; ++t) issue_tile(seq_tile(t) * BN, t);
  dma_next = imin32(kFly + 1, ntiles);

  // Tile classes: each query block's key hull [ulo, uhi] and common interval
  // [ilo, ihi] (classify_tile with the row-dependent parts hoisted).
  int c_ulo[QB], c_uhi[QB], c_ilo[QB], c_ihi[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    c_ulo[qb] = __builtin_amdgcn_readlane(lk[qb][0], wave);
    c_uhi[qb] = __builtin_amdgcn_readlane(lk[qb][1], wave);
    c_ilo[qb] = __builtin_amdgcn_readlane(lk[qb][2], wave);
    c_ihi[qb] = __builtin_amdgcn_readlane(lk[qb][3], wave);
  }
  auto tile_class = [&](int qb, int c, int d) {
    if (!valid[qb]) return (int)TILE_EMPTY;
    const bool tail = d > g.S - 1;
    if (!tail && d < g.prefix) return (int)TILE_FULL;
    if (c_ulo[qb] > c_uhi[qb] || c > c_uhi[qb] || d < c_ulo[qb]) return c < g.prefix ? (int)TILE_PARTIAL : (int)TILE_EMPTY;
    if (!tail && c >= c_ilo[qb] && d <= c_ihi[qb]) return (int)TILE_FULL;
    return (int)TILE_PARTIAL;
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

  // Per-lane LDS byte offsets.  K fragment (kb, kk): row 32 kb + lq, chunk
  // 2 kk + lh -> byte (32 kb) RP + [k_lane ^ 32 kk].
  const int k_lane = lq * RP + 16 * k_slot<D>(lq, lh);
  // V transposed read (c, rr, db): lane (group g16, slot s16) addresses row
  // 16 c + 8 rr + 4 (g16 / 2) + s16 / 4 and elements 32 db + 16 (g16 % 2) +
  // 4 (s16 % 4) .. +3, i.e. byte (16 c + 8 rr) RP + [v_lane ^ 64 db].
  const int g16 = lane >> 4, s16 = lane & 15;
  const int v_row = 4 * (g16 >> 1) + (s16 >> 2);
  const int v_lane = K_BYTES + v_row * RP + 16 * v_slot<D>(v_row, 2 * (g16 & 1) + ((s16 & 3) >> 1)) + 8 * (s16 & 1);

  // One tile for this wavefront, as a set of 32 x 32 score blocks ("streams"):
  //   PAIR (WIDE = false): four streams, query blocks {0, 1} x key blocks
  //     {0, 1}; the K / V fragments of a key block serve both query blocks;
  //   WIDE: two streams, query block 1 x key blocks {0, 1} -- a tile that only
  //     block 1 sees (a zigzag pair past the light block's diagonal).
  // All QK^T MFMAs of the tile are issued before the softmax needs their
  // results, and each query block's row state (m, l) takes one joint update
  // per tile, so the only branch between the first MFMA and the last one is
  // the (rare) rescale.  masked[qb] selects the per-element predicate for a
  // block the tile only partly covers.
  //   WIDE2: four streams, query block 1 x the four key blocks of two
  //     consecutive tiles (St, St2) -- two WIDE tiles behind one barrier.
  auto tile_step = [&](const char* St, const char* St2, int jt0, const bool* masked, auto mode_tag) {
    constexpr int MODE = decltype(mode_tag)::value;  // 0 PAIR, 1 WIDE, 2 WIDE2
    constexpr bool WIDE = MODE != 0;
    constexpr int NSTR = MODE == 1 ? 2 : 4;
    constexpr int NKB = MODE == 2 ? 2 * KB : KB;  // key blocks of the step
    auto qb_of = [](int st) { return WIDE ? 1 : (st & 1); };
    auto kb_of = [](int st) { return WIDE ? st : (st >> 1); };
    // key block kb (0 .. NKB-1) of the step: its stage and first row there
    auto kb_base = [&](int kb) { return (kb < KB ? St : St2) + 32 * (kb % KB) * RP; };
    f32x16_t sacc[NSTR];
    float bias0[NSTR];  // ALiBi softmax: bq (j0 - i) of the stream's block (scores are sacc + bias0)
#pragma unroll
    for (int st = 0; st < NSTR; ++st) {
      if constexpr (kBiasFold) {
        bias0[st] = bq * (float)(jt0 + 32 * kb_of(st) + 4 * lh - (row0[qb_of(st)] + lq));
        sacc[st] = bias_rc;
      } else if constexpr (kBiasInit) {
        bias0[st] = 0.f;
        const float b0 = bq * (float)(jt0 + 32 * kb_of(st) + 4 * lh - (row0[qb_of(st)] + lq));
#pragma unroll
        for (int e = 0; e < 16; ++e) sacc[st][e] = __builtin_fmaf(bq, (float)(8 * (e >> 2) + (e & 3)), b0);
      } else {
        bias0[st] = 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) sacc[st][e] = 0.f;
      }
    }

    // S^T = K Q^T, key block by key block.  For plain softmax the wavefront
    // issues its MFMAs (here and in PV) at raised priority, so that the
    // SIMD's other wavefront fills the matrix core's busy cycles with its
    // vector work rather than delaying them (measured: 2-3% on the causal
    // softmax variants; slower for the modifiers and the pipelined kernels).
    if constexpr (kPlainSoftmax) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
      for (int kk = 0; kk < DK; ++kk) {
        const bf16x8_t a = *(const bf16x8_t*)(kb_base(kb) + (k_lane ^ (32 * kk)));
#pragma unroll
        for (int st = 0; st < NSTR; ++st)
          if (kb_of(st) == kb)
            sacc[st] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[qb_of(st)][kk], sacc[st], 0, 0, 0);
      }
    }

    if constexpr (kPlainSoftmax) __builtin_amdgcn_s_setprio(0);
    // score modifier -> t (in place)
    if constexpr (!kScaledSoftmax && !kRawRelu && !kSigFold) {
#pragma unroll
      for (int st = 0; st < NSTR; ++st) {
        const int i = row0[qb_of(st)] + lq;
        const int jbase = jt0 + 32 * kb_of(st) + 4 * lh;
        const float ksb = ALIBI ? ks * (float)(jbase - i) + k0 : k0;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int rc = 8 * (e >> 2) + (e & 3);  // key offset of register e
          const float qk = sacc[st][e];
          float lin;
          if constexpr (ALIBI && !kBiasInit) lin = __builtin_fmaf(qk, kq, __builtin_fmaf(ks, (float)rc, ksb));
          else if constexpr (NORM == NORM_SIGMOID && !SOFTCAP) lin = __builtin_fmaf(qk, kq, k0);
          else lin = qk * kq;
          if constexpr (kCapR) {
            sacc[st][e] = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(lin));
          } else if constexpr (SOFTCAP) {
            const float u = __builtin_amdgcn_exp2f(lin);
            sacc[st][e] = __builtin_fmaf(__builtin_amdgcn_rcpf(1.0f + u), sc_a, sc_b);
          } else {
            sacc[st][e] = lin;
          }
        }
      }
    }
    // mask (PARTIAL tiles only): softmax/ReLU -> -inf, sigmoid input -> +inf; all give p = 0
    if (masked[0] || masked[1]) {
#pragma unroll
      for (int st = 0; st < NSTR; ++st) {
        if (masked[qb_of(st)]) {
          // the row's key interval is recomputed here rather than kept live
          // (the opaque row index keeps the compiler from hoisting it out of
          // the tile loop, where the pipelined ReLU kernel spilled it)
          int i = row0[qb_of(st)] + lq;
          asm volatile("" : "+v"(i));
          const int jbase = jt0 + 32 * kb_of(st) + 4 * lh;
          const uint32_t hidden = hidden_bits(g, i, jbase);  // bit k: key jbase + k hidden from row i
          // the +-inf pattern in an SGPR (loaded opaquely, so the blend below
          // stays one three-input bitwise op instead of xor + op with a literal)
          uint32_t hide_bits;
          asm("s_mov_b32 %0, %1" : "=s"(hide_bits) : "i"((NORM == NORM_SIGMOID || kCapR) ? 0x7f800000 : 0xff800000));
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int rc = 8 * (e >> 2) + (e & 3);
            // all ones where hidden (v_bfe_i32), then a bitwise blend of the +-inf pattern
            uint32_t m = (uint32_t)__builtin_amdgcn_sbfe((int)hidden, rc, 1);
            asm("" : "+v"(m));  // keeps the blend bitwise instead of compare + select
            sacc[st][e] = __uint_as_float((m & hide_bits) | (~m & __float_as_uint(sacc[st][e])));
          }
        }
      }
    }

    // normaliser -> p, packed to bf16 pairs (pk[st][w] holds registers 2w, 2w+1)
    uint32_t pk[NSTR][8];
    if constexpr (NORM == NORM_SOFTMAX) {
      // Weights against the running reference max: p = 2^(t - m).  The
      // tile's own max is only computed when a row has no reference yet or a
      // lane's partial row sum over the tile exceeds kLazyBound: then some
      // weight may exceed it, the reference moves to the tile's max and the
      // tile's weights are recomputed.  Otherwise every p <= kLazyBound.
      auto exps = [&](float* lt) __attribute__((always_inline)) {
#pragma unroll
        for (int st = 0; st < NSTR; ++st) {
          const int qb = qb_of(st);
          const float m_use = (m_run[qb] == -INFINITY) ? 0.f : m_run[qb];
          const float moff = kBiasFold ? __builtin_fmaf(bias0[st], kq, -m_use) : -m_use;
          float ls = lt[qb];
#pragma unroll
          for (int w = 0; w < 8; ++w) {
            float p0, p1;
            if constexpr (kScaledSoftmax) {
              p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[st][2 * w], kq, moff));
              p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[st][2 * w + 1], kq, moff));
            } else if constexpr (kCapR) {
              p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[st][2 * w], sc_a, sc_b - m_use));
              p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[st][2 * w + 1], sc_a, sc_b - m_use));
            } else {
              p0 = __builtin_amdgcn_exp2f(sacc[st][2 * w] - m_use);
              p1 = __builtin_amdgcn_exp2f(sacc[st][2 * w + 1] - m_use);
            }
            const bf16x2_t pb = pack2(p0, p1);
            ls = __builtin_amdgcn_fdot2_f32_bf16(pb, kOnes2, ls, false);  // row sum of the bf16 weights
            pk[st][w] = __builtin_bit_cast(uint32_t, pb);
          }
          lt[qb] = ls;
        }
      };
      float lt[QB] = {0.f, 0.f};
      // wavefront-uniform decision: every lane takes the same path
      bool fresh = !kLazyMax;  // the exact path: always without the lazy max, else for rows without a reference
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
        if (!(WIDE && qb == 0)) fresh |= m_run[qb] == -INFINITY;
      bool exact = __any(fresh);
      if (!exact) {
        exps(lt);
        bool big = false;
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
          if (!(WIDE && qb == 0)) big |= !(lt[qb] <= kLazyBound);
        exact = __any(big);
      }
      if (exact) {
        // joint row max over the tile's key blocks of each query block
        float mq[QB] = {-INFINITY, -INFINITY};
#pragma unroll
        for (int st = 0; st < NSTR; ++st) {
          float mx = sacc[st][0];
          if constexpr (kCapR) {  // t = sc_a r + sc_b with sc_a < 0: max t <-> min r
#pragma unroll
            for (int e = 1; e < 16; ++e) mx = fminf(mx, sacc[st][e]);
            mx = __builtin_fmaf(mx, sc_a, sc_b);
          } else {
#pragma unroll
            for (int e = 1; e < 16; ++e) mx = fmaxf(mx, sacc[st][e]);
            if constexpr (kBiasFold) mx += bias0[st];
          }
          mq[qb_of(st)] = fmaxf(mq[qb_of(st)], mx);
        }
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          if (WIDE && qb == 0) continue;
          float mx = xhalf_max(mq[qb]);
          if constexpr (kScaledSoftmax) mx = mx * kq;  // kq > 0
          const float m_new = (mx > m_run[qb] + kRescaleLog2) ? mx : m_run[qb];
          if (m_new != m_run[qb]) {  // per lane: the row's O and l follow its reference
            const float alpha = (m_run[qb] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run[qb] - m_new);
            l_run[qb] *= alpha;
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
              for (int e = 0; e < 16; ++e) oacc[db][qb][e] *= alpha;
            m_run[qb] = m_new;
          }
          lt[qb] = 0.f;
        }
        exps(lt);
      }
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
        if (!(WIDE && qb == 0)) l_run[qb] += lt[qb];
    } else {
#pragma unroll
      for (int st = 0; st < NSTR; ++st) {
#pragma unroll
        for (int w = 0; w < 8; ++w) {
          float p0 = sacc[st][2 * w], p1 = sacc[st][2 * w + 1];
          if constexpr (kSigFold) {
            p0 = __builtin_amdgcn_rcpf(__builtin_fmaf(sig_c, __builtin_amdgcn_exp2f(p0), 1.0f));
            p1 = __builtin_amdgcn_rcpf(__builtin_fmaf(sig_c, __builtin_amdgcn_exp2f(p1), 1.0f));
          } else if constexpr (NORM == NORM_SIGMOID) {
            p0 = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(p0));
            p1 = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(p1));
          } else {
            p0 = relu0(p0);
            p1 = relu0(p1);
          }
          pk[st][w] = __builtin_bit_cast(uint32_t, pack2(p0, p1));
        }
      }
    }

    // O^T += V^T P^T, 16-key chunk by chunk
    typedef short i16x8_t __attribute__((ext_vector_type(8)));
    static_assert(DB % 2 == 0, "d-blocks are read in pairs");
    if constexpr (kPlainSoftmax) __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int c = 0; c < 2 * NKB; ++c) {
      const int kb = c >> 1, half = c & 1;
#pragma unroll
      for (int db = 0; db < DB; db += 2) {
        const char* va = kb_base(kb) + 16 * half * RP + (v_lane ^ (64 * db));
        const char* vb = kb_base(kb) + 16 * half * RP + (v_lane ^ (64 * (db + 1)));
        const i16x4_t lo0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)va);
        const i16x4_t hi0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(va + 8 * RP));
        const i16x4_t lo1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)vb);
        const i16x4_t hi1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(vb + 8 * RP));
        const bf16x8_t a0 = __builtin_bit_cast(bf16x8_t, (i16x8_t)__builtin_shufflevector(lo0, hi0, 0, 1, 2, 3, 4, 5, 6, 7));
        const bf16x8_t a1 = __builtin_bit_cast(bf16x8_t, (i16x8_t)__builtin_shufflevector(lo1, hi1, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int st = 0; st < NSTR; ++st) {
          if (kb_of(st) != kb) continue;
          const int qb = qb_of(st);
          const u32x4_t w = {pk[st][4 * half], pk[st][4 * half + 1], pk[st][4 * half + 2], pk[st][4 * half + 3]};
          const bf16x8_t pf = __builtin_bit_cast(bf16x8_t, w);
          oacc[db][qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, pf, oacc[db][qb], 0, 0, 0);
          oacc[db + 1][qb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, pf, oacc[db + 1][qb], 0, 0, 0);
        }
      }
    }
    if constexpr (kPlainSoftmax) __builtin_amdgcn_s_setprio(0);
  };

  // ---- main loop -------------------------------------------------------------
  // Band tiles whose class is known without classifying (both blocks FULL,
  // or block 0 done and block 1 FULL); everything else is classified.
  const FastRanges fr{__builtin_amdgcn_readlane(lf.pf_lo, wave), __builtin_amdgcn_readlane(lf.pf_hi, wave),
                      __builtin_amdgcn_readlane(lf.wf_lo, wave), __builtin_amdgcn_readlane(lf.wf_hi, wave)};
  // WIDE2 tiles: block 0 done and block 1 FULL in every wavefront, since a
  // WIDE2 step changes the barrier count (wide_range_all, from the lanes).
  TileSpan w2{1, 0};
  if constexpr (kWide2) {
    w2 = TileSpan{0, 0x7fffffff};
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      w2.lo = imax32(w2.lo, __builtin_amdgcn_readlane(lf.wf_lo, w));
      w2.hi = imin32(w2.hi, __builtin_amdgcn_readlane(lf.wf_hi, w));
    }
  }

  // ---- pipelined run over the tiles both blocks see in full -----------------
  // A step is one 32-key block kb of a tile for both query blocks (two 32 x 32
  // score blocks).  With step c pending (its scores in a register buffer),
  // step n runs as: QK^T MFMAs of n beside the exponentials of c, then PV of c
  // beside the score modifier and row max of n, then the (rare) rescale for
  // n.  Steps alternate between two score buffers: kb 0 steps use buffer 0,
  // kb 1 steps buffer 1, so the buffer of each step is known at compile time.
  auto p_qk = [&](const char* St, int kb, f32x16_t* sa) __attribute__((always_inline)) {
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int e = 0; e < 16; ++e) sa[st][e] = 0.f;
#pragma unroll
    for (int kk = 0; kk < DK; ++kk) {
      const bf16x8_t a = *(const bf16x8_t*)(St + 32 * kb * RP + (k_lane ^ (32 * kk)));
      sa[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[0][kk], sa[0], 0, 0, 0);
      sa[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[1][kk], sa[1], 0, 0, 0);
    }
  };
  auto p_score = [&](int jt0, int kb, f32x16_t* sa, float* mx) __attribute__((always_inline)) {
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      if constexpr (!kPlainSoftmax && !kRawRelu && !kSigFold) {
        const int i = row0[st] + lq;
        const int jbase = jt0 + 32 * kb + 4 * lh;
        const float ksb = ALIBI ? ks * (float)(jbase - i) + k0 : k0;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int rc = 8 * (e >> 2) + (e & 3);
          const float qkv = sa[st][e];
          float lin;
          if constexpr (ALIBI) lin = __builtin_fmaf(qkv, kq, __builtin_fmaf(ks, (float)rc, ksb));
          else if constexpr (NORM == NORM_SIGMOID && !SOFTCAP) lin = __builtin_fmaf(qkv, kq, k0);
          else lin = qkv * kq;
          if constexpr (SOFTCAP) {
            const float u = __builtin_amdgcn_exp2f(lin);
            sa[st][e] = __builtin_fmaf(__builtin_amdgcn_rcpf(1.0f + u), sc_a, sc_b);
          } else {
            sa[st][e] = lin;
          }
        }
      }
      if constexpr (NORM == NORM_SOFTMAX) {
        float m = sa[st][0];
#pragma unroll
        for (int e = 1; e < 16; ++e) m = fmaxf(m, sa[st][e]);
        mx[st] = m;
      }
    }
  };
  auto p_update = [&](const float* mx) __attribute__((always_inline)) {
    if constexpr (NORM == NORM_SOFTMAX) {
      float m_new[QB];
      bool moved = false;
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        float m = xhalf_max(mx[qb]);
        if constexpr (kPlainSoftmax) m = m * kq;  // kq > 0
        m_new[qb] = (m > m_run[qb] + kRescaleLog2) ? m : m_run[qb];
        moved |= m_new[qb] != m_run[qb];
      }
      if (__any(moved)) {
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          const float alpha = (m_run[qb] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run[qb] - m_new[qb]);
          l_run[qb] *= alpha;
#pragma unroll
          for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int e = 0; e < 16; ++e) oacc[db][qb][e] *= alpha;
        }
      }
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) m_run[qb] = m_new[qb];
    }
  };
  auto p_expo = [&](f32x16_t* sa, uint32_t (*pk)[8]) __attribute__((always_inline)) {
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      if constexpr (NORM == NORM_SOFTMAX) {
        const float m_use = (m_run[st] == -INFINITY) ? 0.f : m_run[st];
        float ls = l_run[st];
#pragma unroll
        for (int w = 0; w < 8; ++w) {
          float p0, p1;
          if constexpr (kPlainSoftmax) {
            p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sa[st][2 * w], kq, -m_use));
            p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sa[st][2 * w + 1], kq, -m_use));
          } else {
            p0 = __builtin_amdgcn_exp2f(sa[st][2 * w] - m_use);
            p1 = __builtin_amdgcn_exp2f(sa[st][2 * w + 1] - m_use);
          }
          const bf16x2_t pb = pack2(p0, p1);
          ls = __builtin_amdgcn_fdot2_f32_bf16(pb, kOnes2, ls, false);
          pk[st][w] = __builtin_bit_cast(uint32_t, pb);
        }
        l_run[st] = ls;
      } else {
#pragma unroll
        for (int w = 0; w < 8; ++w) {
          float p0 = sa[st][2 * w], p1 = sa[st][2 * w + 1];
          if constexpr (kSigFold) {
            p0 = __builtin_amdgcn_rcpf(__builtin_fmaf(sig_c, __builtin_amdgcn_exp2f(p0), 1.0f));
            p1 = __builtin_amdgcn_rcpf(__builtin_fmaf(sig_c, __builtin_amdgcn_exp2f(p1), 1.0f));
          } else if constexpr (NORM == NORM_SIGMOID) {
            p0 = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(p0));
            p1 = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(p1));
          } else {
            p0 = relu0(p0);
            p1 = relu0(p1);
          }
          pk[st][w] = __builtin_bit_cast(uint32_t, pack2(p0, p1));
        }
      }
    }
  };
  // PV of one 16-key half of a step (weights pk[.][4 half .. 4 half + 3]).
  auto p_pv = [&](const char* St, int kb, uint32_t (*pk)[8], int half) __attribute__((always_inline)) {
    typedef short i16x8_t __attribute__((ext_vector_type(8)));
    {
      const int c = 2 * kb + half;
      bf16x8_t pf[2];
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const u32x4_t w = {pk[st][4 * half], pk[st][4 * half + 1], pk[st][4 * half + 2], pk[st][4 * half + 3]};
        pf[st] = __builtin_bit_cast(bf16x8_t, w);
      }
#pragma unroll
      for (int db = 0; db < DB; db += 2) {
        const char* va = St + 16 * c * RP + (v_lane ^ (64 * db));
        const char* vb = St + 16 * c * RP + (v_lane ^ (64 * (db + 1)));
        const i16x4_t lo0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)va);
        const i16x4_t hi0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(va + 8 * RP));
        const i16x4_t lo1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)vb);
        const i16x4_t hi1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(vb + 8 * RP));
        const bf16x8_t a0 = __builtin_bit_cast(bf16x8_t, (i16x8_t)__builtin_shufflevector(lo0, hi0, 0, 1, 2, 3, 4, 5, 6, 7));
        const bf16x8_t a1 = __builtin_bit_cast(bf16x8_t, (i16x8_t)__builtin_shufflevector(lo1, hi1, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int st = 0; st < 2; ++st) {
          oacc[db][st] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, pf[st], oacc[db][st], 0, 0, 0);
          oacc[db + 1][st] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, pf[st], oacc[db + 1][st], 0, 0, 0);
        }
      }
    }
  };
  // One step with step c pending in sb[P]; the new step goes to sb[1 - P].
  // ReLU defers the second 16-key half of a step's PV to the next body (its
  // weights stay in pk[.][4..7] until then): measured 1-2 % faster for ReLU,
  // neutral to 1 % slower for sigmoid, whose body keeps both halves.
  constexpr bool kDefer = NORM == NORM_RELU;
  auto p_body = [&](f32x16_t (*sb)[2], uint32_t (*pk)[8], auto ptag, auto dtag, const char* Sd, int kbd,
                    const char* Sc, int kbc, const char* Sn, int jtn, int kbn) __attribute__((always_inline)) {
    constexpr int P = decltype(ptag)::value;
    if constexpr (kDefer && decltype(dtag)::value) p_pv(Sd, kbd, pk, 1);
    p_qk(Sn, kbn, sb[1 - P]);
    p_expo(sb[P], pk);
    p_pv(Sc, kbc, pk, 0);
    if constexpr (!kDefer) p_pv(Sc, kbc, pk, 1);
    float mx[2];
    p_score(jtn, kbn, sb[1 - P], mx);
    p_update(mx);
  };
  // Iterations [ia, ib) of tiles both blocks see in full, ib > ia.
  auto run_pipelined = [&](int ia, int ib) __attribute__((always_inline)) {
    f32x16_t sb[2][2];
    uint32_t pk[2][8];
    sync_tile(ia);
    const char* S0 = lds + (ia & (NS - 1)) * STAGE_BYTES;
    const int j0 = seq_tile(ia) * BN;
    {
      float mx[2];
      p_qk(S0, 0, sb[0]);
      p_score(j0, 0, sb[0], mx);
      p_update(mx);
    }
    p_body(sb, pk, IntTag<0>{}, BoolTag<false>{}, S0, 0, S0, 0, S0, j0, 1);
    const char* Sp = S0;
    for (int it = ia + 1; it < ib; ++it) {
      sync_tile(it);
      const char* St = lds + (it & (NS - 1)) * STAGE_BYTES;
      const int jt0 = seq_tile(it) * BN;
      // (a deferred half reads the previous tile, which the DMA only
      // overwrites after the next barrier: oldest = it - 1)
      p_body(sb, pk, IntTag<1>{}, BoolTag<true>{}, Sp, 0, Sp, 1, St, jt0, 0);
      p_body(sb, pk, IntTag<0>{}, BoolTag<true>{}, Sp, 1, St, 0, St, jt0, 1);
      Sp = St;
    }
    if constexpr (kDefer) p_pv(Sp, 0, pk, 1);
    p_expo(sb[1], pk);
    p_pv(Sp, 1, pk, 0);
    p_pv(Sp, 1, pk, 1);
  };
  // The pipelined run covers the band tiles of [fr.pf_lo, fr.pf_hi].
  int ia = ntiles, ib = ntiles;
  if constexpr (kPipe) {
    const int lo = imax32(fr.pf_lo, tr.start2), hi = imin32(fr.pf_hi, tr.start2 + tr.n2 - 1);
    if (lo <= hi) {
      ia = tr.n_pre + (lo - tr.start2);
      ib = tr.n_pre + (hi - tr.start2) + 1;
    }
  }

  for (int it = 0; it < ntiles; ++it) {
    if constexpr (kPipe) {
      if (it == ia) {
        run_pipelined(ia, ib);
        it = ib - 1;
        continue;
      }
    }
    const int jt0 = seq_tile(it) * BN;
    // Two consecutive tiles that only block 1 sees, both in full: one WIDE2
    // step behind one barrier.
    if constexpr (kWide2) {
      const int t = jt0 / BN;
      if constexpr (kRev) {  // tiles t, t - 1
        if (in_band(it) && in_band(it + 1) && t - 1 >= w2.lo && t <= w2.hi) {
          sync_step(it, 2, it);
          const bool none[QB] = {false, false};
          tile_step(lds + ((it + 1) & (NS - 1)) * STAGE_BYTES, lds + (it & (NS - 1)) * STAGE_BYTES, jt0 - BN, none,
                    IntTag<2>{});
          ++it;
          continue;
        }
      } else if (it >= tr.n_pre && it + 1 < ntiles && t >= w2.lo && t + 1 <= w2.hi) {
        sync_step(it, 2, it);
        const bool none[QB] = {false, false};
        tile_step(lds + (it & (NS - 1)) * STAGE_BYTES, lds + ((it + 1) & (NS - 1)) * STAGE_BYTES, jt0, none, IntTag<2>{});
        ++it;
        continue;
      }
    }
    sync_tile(it);
    const char* St = lds + (it & (NS - 1)) * STAGE_BYTES;
    int act = 0;
    bool masked[QB] = {false, false};
    const int t = jt0 / BN;
    if (in_band(it) && t >= fr.pf_lo && t <= fr.pf_hi) {
      act = 3;
    } else if (in_band(it) && t >= fr.wf_lo && t <= fr.wf_hi) {
      act = 2;
    } else {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        const int cls = tile_class(qb, jt0, jt0 + BN - 1);
        act |= (cls != TILE_EMPTY) << qb;
        masked[qb] = cls == TILE_PARTIAL;
      }
    }
    // Two code paths: both blocks (PAIR), or only block 1 (WIDE: the common
    // case of a zigzag pair past the light block's diagonal).  A tile that
    // only block 0 sees runs the PAIR path with block 1 fully masked.
    if (act == 2) {
      tile_step(St, St, jt0, masked, IntTag<1>{});
    } else if (act != 0) {
      masked[1] = masked[1] || act == 1;
      tile_step(St, St, jt0, masked, IntTag<0>{});
    }
  }

  // ---- epilogue: normalise and store ----------------------------------------
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const int i = row0[qb] + lq;
    float f;
    if constexpr (NORM == NORM_SOFTMAX) {
      const float lt = xhalf_sum(l_run[qb]);
      f = lt > 0.f ? 1.0f / lt : 0.f;
      // log-sum-exp of the row's (modified) scores, natural log: the weights
      // summed into l are 2^(t log2 e - m), so LSE = (m + log2 l) ln 2
      // (-inf for a row that sees no key)
      if (p.lse != nullptr && lh == 0 && valid[qb] && i < g.S) {
        const float lse2 = lt > 0.f ? m_run[qb] + __builtin_amdgcn_logf(lt) : -INFINITY;
        p.lse[b * p.lse_sb + h * p.lse_sh + (t0 + (int64_t)g.dil * i) * p.lse_ss] = lse2 * kLn2;
      }
    } else {
      f = post;
    }
    if (valid[qb] && i < g.S) {
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
