// attn_fwd_q1_kernel.h -- the one-block forward core: one 32-row query block
// per wavefront.  It runs every head_dim 128 forward but long full rows of
// sigmoid / ReLU, and at head_dim 64 the banded masks (window, block), causal
// rows with a prefix, and causal softmax on large grids.
//
// Reference semantics: the eager closures of extra_bench.py:32-62 and
// sigmoid_fix.py:34-40, as for attn_fwd_kernel.h, whose helpers (DMA, LDS
// layout, score constants, masks, packing) this kernel shares.
//
// Why a second core.
//   * head_dim 128: the paired core (two query blocks per wavefront) holds 128
//     accumulator registers of O alone and runs one wavefront per SIMD, so
//     nothing hides its softmax behind another wavefront's MFMAs.  One query
//     block per wavefront needs ~180 VGPRs (no spills), two wavefronts fit on
//     each SIMD, and the SIMD interleaves them.  The paired core keeps the
//     case where it measured faster: sigmoid and ReLU on full rows (no causal
//     pairing, window or block) of 2048 keys or more without a score
//     modifier, where sharing each K/V tile between two row blocks halves the
//     K/V reads.
//   * head_dim 64, banded masks: a workgroup's key range is its rows plus the
//     window, a few tiles; four wavefronts per SIMD (103-126 VGPRs) hide the
//     latency of those few tiles better than the paired core's two.  Causal
//     rows (a prefix, or softmax on large grids): one block per workgroup,
//     launched longest-first, balances them where zigzag pairs measured slower.
//
// Work decomposition
//   * a workgroup of 4 wavefronts owns row blocks of 128 rows of one (batch,
//     head, dilation residue); each wavefront owns 32 of them (one query
//     block, ONE MFMA stream);
//   * for a causal band without a window (zigzag), a workgroup processes
//     block i and then block n-1-i, one after the other, so every workgroup
//     does the same work; otherwise one block;
//   * the K / V tiles (64 keys) of the block's key range go HBM -> LDS with
//     global_load_lds_dwordx4 through NS stages (one barrier per tile); the
//     DMA runs across the boundary between the two blocks of a pair;
//   * a tile is computed as two 32-key steps: S^T = K Q^T (D / 16 MFMAs),
//     score modifier, mask on partial steps, normaliser with its own row-max
//     update (lazy at head_dim 64), then O^T += V^T P^T (D / 16 MFMAs), with
//     the matrix-core layouts of the paired core (lane = query column; V^T
//     read with ds_read_b64_tr_b16); a 32-key step that no row of the
//     wavefront sees is skipped.
#pragma once
#include "attn_fwd_kernel.h"

namespace chia {

// Waves per SIMD the register budget targets, and LDS stages per workgroup:
// head_dim 64, four workgroups per CU x 2 stages x 16 KB; head_dim 128, two
// workgroups per CU x 2 stages x 32 KB.
template <int D>
struct Q1Config {
  static_assert(D == 64 || D == 128, "head_dim 64 or 128");
  static constexpr int occupancy = D == 64 ? 4 : 2;
  static constexpr int stages = 2;
};

// NG = 2: the workgroup holds two groups of four wavefronts that split one
// zigzag pair's steps between them (below); NG = 1: one group.  CAPFIX
// (softcap softmax with cap log2 e <= 78, chosen by the host): the weights are
// taken against a fixed reference (below) instead of a running max.
template <int D, int NORM, bool ALIBI, bool SOFTCAP, int NG = 1, bool CAPFIX = false>
__global__ __launch_bounds__(256 * NG, Q1Config<D>::occupancy) void attn_fwd_q1_kernel(const FwdParams p) {
  static_assert(NG == 1 || NG == 2, "one or two groups");
  static_assert(!CAPFIX || (SOFTCAP && NORM == NORM_SOFTMAX), "the fixed reference is for softcap softmax");
  constexpr int NW = 4;  // wavefronts per group
  constexpr int BN = kBN;
  constexpr int NT = NW * 64;
  constexpr int BM = NW * 32;          // rows per block
  constexpr int DK = D / 16;           // k-steps of the QK^T MFMA
  constexpr int DB = D / 32;           // 32-row d blocks of O^T
  constexpr int DQ = D / 8;            // 16-byte chunks per K/V row
  constexpr int RP = 2 * D;            // LDS row pitch (bytes)
  constexpr int NDMA = BN * DQ / NT;   // 1 KB DMA loads per wavefront per tile (each of K, V)
  constexpr int K_BYTES = BN * RP;
  constexpr int STAGE_BYTES = 2 * K_BYTES;
  constexpr int NS = Q1Config<D>::stages;
  static_assert(NDMA >= 1 && BN * DQ % NT == 0, "tile does not split into whole DMA loads");
  static_assert(RP % 128 == 0, "rows must be whole multiples of 128 bytes for the XOR offsets");
  static_assert(DB % 2 == 0, "d-blocks are read in pairs");
  constexpr bool kPlainSoftmax = (NORM == NORM_SOFTMAX) && !ALIBI && !SOFTCAP;
  constexpr bool kBiasInit = ALIBI && !SOFTCAP;
  constexpr bool kScaledSoftmax = kPlainSoftmax || (kBiasInit && NORM == NORM_SOFTMAX);
  // the step's bias in the exponent (below): ALiBi softmax at head dim 128
  constexpr bool kBiasFold = kBiasInit && NORM == NORM_SOFTMAX && D == 128;
  constexpr bool kRawRelu = (NORM == NORM_RELU) && !ALIBI && !SOFTCAP;
  constexpr bool kCapR = SOFTCAP && NORM == NORM_SOFTMAX;
  constexpr bool kSigFold = NORM == NORM_SIGMOID && !ALIBI && !SOFTCAP;
  __shared__ __attribute__((aligned(1024))) char lds_all[NG * NS * STAGE_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave_wg = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = NG == 2 ? wave_wg >> 2 : 0;  // this wavefront's group
  const int wave = wave_wg & (NW - 1);          // and its index in the group
  char* const lds = lds_all + grp * (NS * STAGE_BYTES);  // the group's LDS stages
  const int lq = lane & 31, lh = lane >> 5;

  // ---- workgroup -> (batch, head, residue, unit) ----------------------------
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
  const int nblk = (g.S + BM - 1) / BM;
  int blk0, blk1;
  if (p.zigzag) {
    blk0 = pr;
    blk1 = nblk - 1 - pr;
    if (blk1 < blk0) return;  // whole workgroup, before any barrier
    if (blk1 == blk0) blk1 = -1;
  } else {
    blk0 = pr;
    blk1 = -1;
    if (blk0 >= nblk) return;
  }

  const int dil = p.mask.dil;
  const int64_t t0 = seq.tok0 + r;
  const uint16_t* qh = p.q + b * p.q_sb + h * p.q_sh + t0 * p.q_ss;
  const int hk = udiv(h, p.div_group);
  const uint16_t* kh = p.k + b * p.k_sb + hk * p.k_sh + t0 * p.k_ss;
  const uint16_t* vh = p.v + b * p.v_sb + hk * p.v_sh + t0 * p.v_ss;
  uint16_t* oh = p.o + b * p.o_sb + h * p.o_sh + t0 * p.o_ss;
  const int64_t qrs = p.q_ss * dil, krs = p.k_ss * dil, vrs = p.v_ss * dil, ors = p.o_ss * dil;

  // ---- per-head score constants (as in attn_fwd_kernel) ----------------------
  const float hs = p.head_scale ? p.head_scale[h] : 1.0f;
  const float slope = ALIBI && p.alibi_slopes ? p.alibi_slopes[h] : 0.0f;
  const float c1 = p.scale * hs;
  const float sl = slope * (float)dil;
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
    kq = ALIBI ? c1 : 1.0f;
    ks = sl;
  }
  const float post = kRawRelu ? p.post_scale * c1 : p.post_scale;
  const float bq = kBiasInit ? sl / c1 : 0.f;
  // ALiBi softmax at head dim 128: S starts from bq rc(e), the bias of
  // register e's key offset inside a 32-key step (the same registers for
  // every step); the rest, bq (j0 - i), joins the exponent once per step.
  // (Elsewhere S starts from the whole bias: at head dim 64 the four
  // wavefronts per SIMD leave no registers to spare.)
  f32x16_t bias_rc;
#pragma unroll
  for (int e = 0; e < 16; ++e) bias_rc[e] = kBiasFold ? bq * (float)(8 * (e >> 2) + (e & 3)) : 0.f;
  const float sig_c =
      kSigFold ? __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(__builtin_amdgcn_exp2f(k0)))) : 0.f;

  // ---- the workgroup's steps: the tiles of block 0, then those of block 1 -----
  const TileRange tr0 = tile_range(g, blk0 * BM, imin32(blk0 * BM + BM - 1, g.S - 1), BN);
  const int n0 = tr0.n_pre + tr0.n2;
  TileRange tr1{0, 0, 0};
  if (blk1 >= 0) tr1 = tile_range(g, blk1 * BM, imin32(blk1 * BM + BM - 1, g.S - 1), BN);
  const int nsteps = n0 + tr1.n_pre + tr1.n2;
  // ALiBi softmax walks each block's key tiles (and the two 32-key steps of a
  // tile) from the last to the first: the bias grows with the key index, so
  // a row's max is set on its first step and O is rarely rescaled after it.
  constexpr bool kRev = ALIBI && NORM == NORM_SOFTMAX;
  const int n1 = tr1.n_pre + tr1.n2;
  // A single block's band tiles [a, a + n) are visited in the order
  // a + ((k - a) mod n): tile T comes at step T mod n in every block that
  // reads it.  Neighbouring blocks of a window or block mask (equal n, ranges
  // shifted by BM / BN tiles) then read each shared tile at the same step,
  // while it is still in L2, rather than BM / BN steps apart.  (Full rows
  // start at tile 0, where the order is the identity.)
  const int rot0 = (!kRev && blk1 < 0 && tr0.n_pre == 0 && n0 > 1) ? tr0.start2 % n0 : 0;
  const int a0 = tr0.start2;
  // (a separate early return: folded into the tile_at selects below, the
  // rotation made the compiler keep both TileRange structs in scratch memory)
  auto step_key0 = [&](int s) {
    if (rot0 != 0 && s < n0) return (a0 + s - rot0 + (s < rot0 ? n0 : 0)) * BN;
    return (s < n0 ? tile_at(tr0, kRev ? n0 - 1 - s : s) : tile_at(tr1, kRev ? n1 - 1 - (s - n0) : s - n0)) * BN;
  };

  // ---- the group's steps -------------------------------------------------------
  // NG = 2 (a zigzag pair on a grid of fewer than two workgroups per CU, where
  // one group alone would leave one wavefront per SIMD): the pair's steps split
  // at M = ceil(nsteps / 2), group 0 running [0, M) and group 1 [M, nsteps).
  // Block 1 has at least block 0's steps, so group 0 computes block 0 whole
  // and block 1's first steps, group 1 the rest of block 1 (of block 0 when
  // there is no block 1).  The block both groups compute part of is merged at
  // the end through LDS, with the log-sum-exp rescale of the two partial
  // (O, m, l).  Each group streams its own tiles through its own LDS stages;
  // the workgroup barrier of every step is shared, so both groups pass the same
  // number of barriers: the group with fewer steps adds empty ones.
  int M = NG == 2 ? (nsteps + 1) / 2 : nsteps;
  if (NG == 2 && blk1 >= 0 && M < n0) M = n0;  // (not reached for causal pairs)
  const int s_lo = grp == 1 ? M : 0, s_hi = grp == 1 ? nsteps : M;
  const int n_bar = imax32(M, nsteps - M);  // step barriers of each group
  // pass (0: block 0, 1: block 1) that both groups compute part of, or -1
  const int split_pass =
      NG == 2 && M > 0 && M < nsteps ? (blk1 >= 0 ? (M > n0 ? 1 : -1) : 0) : -1;

  uint32_t k_dma[NDMA], v_dma[NDMA];
#pragma unroll
  for (int n = 0; n < NDMA; ++n) {
    const int pos = (n * NW + wave) * 64 + lane;
    const int row = pos / DQ, slot = pos % DQ;
    k_dma[n] = (uint32_t)(2 * ((int64_t)row * krs + 8 * k_slot<D>(row, slot)));
    v_dma[n] = (uint32_t)(2 * ((int64_t)row * vrs + 8 * v_slot<D>(row, slot)));
  }
  // The tile's row base as a 32 x 32 -> 64-bit product: keys are
  // non-negative, and a K / V row step (stride times dilation) is below 2^25
  // elements, so its byte count fits 32 bits.
  static_assert((NS & (NS - 1)) == 0, "the stage index is a mask");
  const uint32_t k_row_bytes = 2u * (uint32_t)krs, v_row_bytes = 2u * (uint32_t)vrs;
  auto issue_step = [&](int s, int jt0) {
    char* kst = lds + ((uint32_t)s & (NS - 1)) * STAGE_BYTES;
    const uint16_t* kt = (const uint16_t*)((const char*)kh + (uint64_t)(uint32_t)jt0 * k_row_bytes);
    const uint16_t* vt = (const uint16_t*)((const char*)vh + (uint64_t)(uint32_t)jt0 * v_row_bytes);
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
  // prologue: the first NS - 1 steps (each barrier issues one more).  With
  // two stages one step is in flight: its first key, found for the DMA, is
  // the compute's key one iteration later (jt_dma).
  static_assert(NS == 2, "one step in flight");
  // The DMA's keys are stepped: within a block a step's first key is the
  // previous step's plus BN (minus BN walking backwards), except at the
  // block's start, at the seam between its prefix and band tiles, and at the
  // rotation's wrap, where step_key0 gives it in full.
  const int dkey = kRev ? -BN : BN;
  const int seam0 = rot0 != 0 ? rot0 : (kRev ? tr0.n2 : tr0.n_pre);
  const int seam1 = n0 + (kRev ? tr1.n2 : tr1.n_pre);
  auto next_break = [&](int s) {  // the first step after s whose key is not stepped
    if (s < seam0) return seam0;
    if (s < n0) return n0;
    if (s < seam1) return seam1;
    return 0x7fffffff;
  };
  int dma_next = s_lo;
  int jt_dma = 0, brk = 0;
  for (; dma_next < s_lo + NS - 1 && dma_next < s_hi; ++dma_next) {
    jt_dma = step_key0(dma_next);
    brk = next_break(dma_next);
    issue_step(dma_next, jt_dma);
  }

  // per-lane LDS byte offsets (as in attn_fwd_kernel)
  const int k_lane = lq * RP + 16 * k_slot<D>(lq, lh);
  const int g16 = lane >> 4, s16 = lane & 15;
  const int v_row = 4 * (g16 >> 1) + (s16 >> 2);
  const int v_lane = K_BYTES + v_row * RP + 16 * v_slot<D>(v_row, 2 * (g16 & 1) + ((s16 & 3) >> 1)) + 8 * (s16 & 1);

  // softmax normaliser: a step's K fragments are read before its QK^T chain,
  // and both MFMA chains issue at raised wave priority, so the SIMD's other
  // wavefront runs its exponentials beside them (sigmoid and ReLU measured
  // slower with either)
  constexpr bool kPrio = NORM == NORM_SOFTMAX;
  // Softcap softmax with cap log2 e <= 78 (cap <= 54; the host checks): a
  // score is below cap log2 e = sc_b, so the fixed reference m = sc_b - 48
  // keeps every weight in (2^(48 - 2 sc_b), 2^48], normal in fp32 and bf16:
  // no max, no vote on the row sum, no rescale.  (With a larger cap a row whose
  // scores all lie near -cap would fall below the normal range.)
  const float m_fix = sc_b - 48.0f;
  int step = s_lo;
  bool merged = false;
#pragma unroll 1
  for (int pass = 0; pass < 2; ++pass) {
    const int blk = pass == 0 ? blk0 : blk1;
    if (blk < 0) break;
    const int nt = pass == 0 ? n0 : tr1.n_pre + tr1.n2;
    // this group's steps of the block: [it_lo, it_hi)
    const int base = pass == 0 ? 0 : n0;
    const int it_lo = imax32(s_lo - base, 0), it_hi = imin32(s_hi - base, nt);
    if (it_lo >= it_hi) continue;
    const int row0 = blk * BM + 32 * wave;
    const bool valid = row0 < g.S;
    const int i = row0 + lq;  // this lane's query row
    bf16x8_t qf[DK];
    {
      const bool ok = valid && i < g.S;
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
        qf[kk] = __builtin_bit_cast(bf16x8_t, val);
      }
    }
    // the class of a 32-key step against this wavefront's rows (mask.h)
    const KeyRanges<32> kr(g, valid, row0, imin32(row0 + 31, g.S - 1));

    f32x16_t oacc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int e = 0; e < 16; ++e) oacc[db][e] = 0.f;
    float m_run = CAPFIX ? m_fix : -INFINITY, l_run = 0.f;

#pragma unroll 1
    for (int it = it_lo; it < it_hi; ++it, ++step) {
      // wait for this step's tile (NS - 2 later steps may stay in flight), then the barrier
      if constexpr (NS >= 3) {
        if (dma_next - (step + 1) >= 1) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * NDMA) : "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      } else {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
      __builtin_amdgcn_s_barrier();
      asm volatile("" ::: "memory");
      const int jt0 = jt_dma;  // this step's first key
      if (dma_next < s_hi) {
        if (dma_next == brk) {
          jt_dma = step_key0(dma_next);
          brk = next_break(dma_next);
        } else {
          jt_dma += dkey;
        }
        issue_step(dma_next, jt_dma);
        ++dma_next;
      }
      const char* St = lds + ((uint32_t)step & (NS - 1)) * STAGE_BYTES;

#pragma unroll
      for (int kbs = 0; kbs < 2; ++kbs) {
        const int kb = kRev ? 1 - kbs : kbs;
        const int jb = jt0 + 32 * kb;
        const int cls = key_class(kr, jb);
        if (cls == TILE_EMPTY) continue;
        const char* Kb = St + 32 * kb * RP;
        f32x16_t s;
        float bias0 = 0.f;  // ALiBi softmax: bq (j0 - i) of this step (scores are s + bias0)
        if constexpr (kBiasFold) {
          bias0 = bq * (float)(jb + 4 * lh - i);
          s = bias_rc;
        } else if constexpr (kBiasInit) {
          const float b0 = bq * (float)(jb + 4 * lh - i);
#pragma unroll
          for (int e = 0; e < 16; ++e) s[e] = __builtin_fmaf(bq, (float)(8 * (e >> 2) + (e & 3)), b0);
        } else {
#pragma unroll
          for (int e = 0; e < 16; ++e) s[e] = 0.f;
        }
        if constexpr (kPrio) {
          __builtin_amdgcn_s_setprio(1);
          bf16x8_t kf[DK];
#pragma unroll
          for (int kk = 0; kk < DK; ++kk) kf[kk] = *(const bf16x8_t*)(Kb + (k_lane ^ (32 * kk)));
#pragma unroll
          for (int kk = 0; kk < DK; ++kk) s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[kk], qf[kk], s, 0, 0, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, DK, 0);  // the DK LDS reads first,
          __builtin_amdgcn_sched_group_barrier(0x008, DK, 0);  // then the DK MFMAs
          __builtin_amdgcn_s_setprio(0);
        } else {
#pragma unroll
          for (int kk = 0; kk < DK; ++kk) {
            const bf16x8_t a = *(const bf16x8_t*)(Kb + (k_lane ^ (32 * kk)));
            s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[kk], s, 0, 0, 0);
          }
        }
        // score modifier -> t (in place)
        if constexpr (!kScaledSoftmax && !kRawRelu && !kSigFold) {
          const int jbase = jb + 4 * lh;
          const float ksb = ALIBI ? ks * (float)(jbase - i) + k0 : k0;
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int rc = 8 * (e >> 2) + (e & 3);
            const float qk = s[e];
            float lin;
            if constexpr (ALIBI && !kBiasInit) lin = __builtin_fmaf(qk, kq, __builtin_fmaf(ks, (float)rc, ksb));
            else if constexpr (NORM == NORM_SIGMOID && !SOFTCAP) lin = __builtin_fmaf(qk, kq, k0);
            else lin = qk * kq;
            if constexpr (kCapR) {
              s[e] = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(lin));
            } else if constexpr (SOFTCAP) {
              const float u = __builtin_amdgcn_exp2f(lin);
              s[e] = __builtin_fmaf(__builtin_amdgcn_rcpf(1.0f + u), sc_a, sc_b);
            } else {
              s[e] = lin;
            }
          }
        }
        if (cls == TILE_PARTIAL) {
          const uint32_t hidden = hidden_bits(g, i, jb + 4 * lh);
          uint32_t hide_bits;
          asm("s_mov_b32 %0, %1" : "=s"(hide_bits) : "i"((NORM == NORM_SIGMOID || kCapR) ? 0x7f800000 : 0xff800000));
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int rc = 8 * (e >> 2) + (e & 3);
            uint32_t m = (uint32_t)__builtin_amdgcn_sbfe((int)hidden, rc, 1);
            asm("" : "+v"(m));
            s[e] = __uint_as_float((m & hide_bits) | (~m & __float_as_uint(s[e])));
          }
        }

        // normaliser -> p, packed to bf16 pairs
        uint32_t pk[8];
        if constexpr (NORM == NORM_SOFTMAX) {
          // head_dim 64: the lazy row max of the paired core.  The step's
          // weights are first taken against the running max m; only when a
          // row has no max yet, or some lane's partial row sum over the step
          // exceeds kLazyBound (a weight may exceed it), is the step's max
          // taken, m raised when it exceeds m by more than kRescaleLog2, and
          // the weights recomputed.  So p <= kLazyBound.  At head_dim 128
          // (two wavefronts per SIMD) the per-step max measured faster.
          constexpr bool kLazy = D == 64;
          // weights of the step against m_use into pk; lt = start + their
          // lane's row sum
          auto exps = [&](float m_use, float start, float& lt) __attribute__((always_inline)) {
            const float moff = kBiasFold ? __builtin_fmaf(bias0, kq, -m_use) : -m_use;
            float ls = start;
#pragma unroll
            for (int w = 0; w < 8; ++w) {
              float p0, p1;
              if constexpr (kScaledSoftmax) {
                p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[2 * w], kq, moff));
                p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[2 * w + 1], kq, moff));
              } else if constexpr (kCapR) {
                p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[2 * w], sc_a, sc_b - m_use));
                p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[2 * w + 1], sc_a, sc_b - m_use));
              } else {
                p0 = __builtin_amdgcn_exp2f(s[2 * w] - m_use);
                p1 = __builtin_amdgcn_exp2f(s[2 * w + 1] - m_use);
              }
              const bf16x2_t pb = pack2(p0, p1);
              ls = __builtin_amdgcn_fdot2_f32_bf16(pb, kOnes2, ls, false);
              pk[w] = __builtin_bit_cast(uint32_t, pb);
            }
            lt = ls;
          };
          float lt = 0.f;
          bool exact = true;
          if constexpr (CAPFIX) {
            exps(m_run, 0.f, lt);  // m_run is the fixed reference
            exact = false;
          } else if constexpr (kLazy) {
            exact = __any(m_run == -INFINITY);
            if (!exact) {
              exps(m_run, 0.f, lt);
              exact = __any(!(lt <= kLazyBound));
            }
          }
          if (exact) {
            float mx = s[0];
            if constexpr (kCapR) {
#pragma unroll
              for (int e = 1; e < 16; ++e) mx = fminf(mx, s[e]);
              mx = __builtin_fmaf(mx, sc_a, sc_b);
            } else {
#pragma unroll
              for (int e = 1; e < 16; ++e) mx = fmaxf(mx, s[e]);
              if constexpr (kBiasFold) mx += bias0;
            }
            mx = xhalf_max(mx);
            if constexpr (kScaledSoftmax) mx = mx * kq;
            const float m_new = (mx > m_run + kRescaleLog2) ? mx : m_run;
            if (__any(m_new != m_run)) {
              const float alpha = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
              l_run *= alpha;
#pragma unroll
              for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int e = 0; e < 16; ++e) oacc[db][e] *= alpha;
              m_run = m_new;
            }
            const float m_use = (m_run == -INFINITY) ? 0.f : m_run;
            exps(m_use, kLazy ? 0.f : l_run, lt);
          }
          l_run = (kLazy || CAPFIX) ? l_run + lt : lt;
        } else {
#pragma unroll
          for (int w = 0; w < 8; ++w) {
            float p0 = s[2 * w], p1 = s[2 * w + 1];
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
            pk[w] = __builtin_bit_cast(uint32_t, pack2(p0, p1));
          }
        }

        // O^T += V^T P^T, 16-key chunk by chunk
        if constexpr (kPrio) __builtin_amdgcn_s_setprio(1);
        typedef short i16x8_t __attribute__((ext_vector_type(8)));
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const u32x4_t w4 = {pk[4 * half], pk[4 * half + 1], pk[4 * half + 2], pk[4 * half + 3]};
          const bf16x8_t pf = __builtin_bit_cast(bf16x8_t, w4);
#pragma unroll
          for (int db = 0; db < DB; db += 2) {
            const char* pa = Kb + 16 * half * RP + (v_lane ^ (64 * db));  // v_lane includes K_BYTES
            const char* pb2 = Kb + 16 * half * RP + (v_lane ^ (64 * (db + 1)));
            const i16x4_t lo0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)pa);
            const i16x4_t hi0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(pa + 8 * RP));
            const i16x4_t lo1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)pb2);
            const i16x4_t hi1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(pb2 + 8 * RP));
            const bf16x8_t a0 = __builtin_bit_cast(bf16x8_t, (i16x8_t)__builtin_shufflevector(lo0, hi0, 0, 1, 2, 3, 4, 5, 6, 7));
            const bf16x8_t a1 = __builtin_bit_cast(bf16x8_t, (i16x8_t)__builtin_shufflevector(lo1, hi1, 0, 1, 2, 3, 4, 5, 6, 7));
            oacc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, pf, oacc[db], 0, 0, 0);
            oacc[db + 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, pf, oacc[db + 1], 0, 0, 0);
          }
        }
        if constexpr (kPrio) __builtin_amdgcn_s_setprio(0);
      }
    }

    // ---- the block both groups computed part of: merge through LDS -------------
    if constexpr (NG == 2) {
      if (pass == split_pass) {
        merged = true;
        for (int k = s_hi - s_lo; k < n_bar; ++k) __builtin_amdgcn_s_barrier();
        // every wavefront is past its last step (no DMA in flight, no stage
        // still read): the stages of both groups hold the merge buffer, per
        // wavefront of group 1 its 16 DB accumulators, m and l, lane-major
        constexpr int FL = 16 * DB + 2;
        float* mb = reinterpret_cast<float*>(lds_all) + wave * (FL * 64) + lane;
        __syncthreads();
        if (grp == 1) {
#pragma unroll
          for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int e = 0; e < 16; ++e) mb[(16 * db + e) * 64] = oacc[db][e];
          mb[(16 * DB) * 64] = m_run;
          mb[(16 * DB + 1) * 64] = l_run;
        }
        __syncthreads();
        if (grp == 1) return;  // group 0 stores the block
        const float m1 = mb[(16 * DB) * 64], l1 = mb[(16 * DB + 1) * 64];
        if constexpr (NORM == NORM_SOFTMAX) {
          // both partials against the larger reference (a row neither group
          // saw keeps m = -inf, O = 0 and l = 0)
          const float mm = fmaxf(m_run, m1);
          const float a0 = m_run == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_run - mm);
          const float a1 = m1 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m1 - mm);
#pragma unroll
          for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int e = 0; e < 16; ++e) oacc[db][e] = __builtin_fmaf(oacc[db][e], a0, mb[(16 * db + e) * 64] * a1);
          l_run = __builtin_fmaf(l_run, a0, l1 * a1);
          m_run = mm;
        } else {
#pragma unroll
          for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int e = 0; e < 16; ++e) oacc[db][e] += mb[(16 * db + e) * 64];
        }
      }
    }

    // ---- epilogue of this block: normalise and store ---------------------------
    float f;
    if constexpr (NORM == NORM_SOFTMAX) {
      const float lt = xhalf_sum(l_run);
      f = lt > 0.f ? 1.0f / lt : 0.f;
      if (p.lse != nullptr && lh == 0 && valid && i < g.S) {
        const float lse2 = lt > 0.f ? m_run + __builtin_amdgcn_logf(lt) : -INFINITY;
        p.lse[b * p.lse_sb + h * p.lse_sh + (t0 + (int64_t)g.dil * i) * p.lse_ss] = lse2 * kLn2;
      }
    } else {
      f = post;
    }
    if (valid && i < g.S) {
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
    }
  }
  if constexpr (NG == 2) {
    if (!merged)
      for (int k = s_hi - s_lo; k < n_bar; ++k) __builtin_amdgcn_s_barrier();
  }
}

}  // namespace chia
