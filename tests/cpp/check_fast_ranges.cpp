// Brute-force check of fast_ranges and wide_range_all (chia_proj_amd/csrc/mask.h)
// against classify_tile: every band key tile the kernel runs without
// classification must have the class the fast path assumes, in every
// wavefront for the workgroup-uniform WIDE span; and of hidden_bits (the
// per-element mask of partial blocks) against visible(); and of KeyRanges
// and RowRanges (the per-step classes from per-block bounds) against
// classify_tile.  Built and run by
// tests/test_mask_fast_ranges.py; exits non-zero on the first mismatch.
#include <cstdio>
#include <initializer_list>

#include "mask.h"

using namespace chia;

// hidden_bits against visible() for every row and 4-aligned key base (the
// kernel's blocks start at a tile + 32 kb + 4 lane-half)
static int check_hidden_bits(long* n) {
  for (int S : {1, 37, 65, 200, 513})
    for (int causal = 0; causal < 2; ++causal)
      for (int w : {0, 1, 5, 64, 129})
        for (int d : {1, 2, 3})
          for (int blk : {0, 33, 128})
            for (int pre : {0, 40, 130}) {
              if (d > 1 && pre > 0) continue;
              const MaskSpec m = make_mask_spec(S, causal, w, d, blk, pre);
              for (int r = 0; r < num_residues(m); ++r) {
                const MaskGeom g = residue_geom(m, r);
                for (int i = 0; i < g.S; ++i)
                  for (int jb = 0; jb < g.S + 32; jb += 4) {
                    const uint32_t h = hidden_bits(g, i, jb);
                    for (int k = 0; k < 32; ++k) {
                      ++*n;
                      if (((h >> k) & 1u) == (uint32_t)visible(g, i, jb + k)) {
                        std::printf("hidden_bits mismatch S=%d c=%d w=%d d=%d blk=%d p=%d r=%d i=%d j=%d\n", S, causal, w,
                                    d, blk, pre, r, i, jb + k);
                        return 1;
                      }
                    }
                  }
              }
            }
  return 0;
}

// query_range against visible(): every row that sees a key of the block lies
// inside the returned span (key blocks of 32 and 64 keys)
static int check_query_range(long* n) {
  for (int S : {1, 37, 65, 200, 513})
    for (int causal = 0; causal < 2; ++causal)
      for (int w : {0, 1, 5, 64, 129})
        for (int d : {1, 2, 3})
          for (int blk : {0, 33, 128})
            for (int pre : {0, 40, 130}) {
              if (d > 1 && pre > 0) continue;
              const MaskSpec m = make_mask_spec(S, causal, w, d, blk, pre);
              for (int r = 0; r < num_residues(m); ++r) {
                const MaskGeom g = residue_geom(m, r);
                // one key: the span is exact (the backward's per-key row mask);
                // keys past the end give an empty span
                for (int j = 0; j < g.S + 40; ++j) {
                  const RowSpan q = query_range(g, j, j);
                  for (int i = 0; i < g.S; ++i) {
                    ++*n;
                    if ((i >= q.lo && i <= q.hi) != visible(g, i, j)) {
                      std::printf("single-key query_range not exact S=%d c=%d w=%d d=%d blk=%d p=%d r=%d i=%d j=%d\n", S,
                                  causal, w, d, blk, pre, r, i, j);
                      return 1;
                    }
                  }
                }
                for (int bk : {32, 64})
                  for (int j0 = 0; j0 < g.S; j0 += bk) {
                    const RowSpan q = query_range(g, j0, j0 + bk - 1);
                    for (int i = 0; i < g.S; ++i) {
                      bool sees = false;
                      for (int j = j0; j < j0 + bk && j < g.S; ++j) sees = sees || visible(g, i, j);
                      ++*n;
                      if (sees && (i < q.lo || i > q.hi)) {
                        std::printf("query_range misses S=%d c=%d w=%d d=%d blk=%d p=%d r=%d j0=%d i=%d span=[%d,%d]\n", S,
                                    causal, w, d, blk, pre, r, j0, i, q.lo, q.hi);
                        return 1;
                      }
                    }
                  }
              }
            }
  return 0;
}

// KeyRanges<N>::classify (the kernels' per-step class from bounds set once
// per row block) against classify_tile for every 32-row block of a wavefront,
// and every key offset c (multiples of 4, past both ends), N = 32 and 64;
// a block without rows is EMPTY everywhere.
template <int N>
static int check_key_ranges_n(const MaskGeom& g, long* n, const char* tag) {
  for (int a = 0; a < g.S + 64; a += 32) {
    const bool valid = a < g.S;
    const int b = imin32(a + 31, g.S - 1);
    const KeyRanges<N> kr(g, valid, a, b);
    for (int c = -2 * N; c < g.S + 2 * N; c += 4) {
      const int want = valid ? classify_tile(g, a, b, c, c + N - 1) : (int)TILE_EMPTY;
      ++*n;
      if (kr.classify(c) != want) {
        std::printf("KeyRanges<%d> mismatch %s a=%d c=%d got %d want %d\n", N, tag, a, c, kr.classify(c), want);
        return 1;
      }
    }
  }
  return 0;
}

// RowRanges<M>::classify (the dK/dV kernel's per-tile class of its query row
// tiles against a wavefront's fixed 32 keys) against classify_tile, for every
// 32-aligned key block and every row tile start of either tile height.
template <int M>
static int check_row_ranges_m(const MaskGeom& g, long* n, const char* tag) {
  for (int c = 0; c < g.S; c += 32) {
    const int d = c + 31;
    for (int valid = 0; valid < 2; ++valid) {
      const RowRanges<M> rr(g, valid != 0, c, d);
      for (int a = 0; a < g.S; a += (M > 32 ? 16 : 8)) {
        const int want = valid ? classify_tile(g, a, imin32(a + M - 1, g.S - 1), c, d) : (int)TILE_EMPTY;
        ++*n;
        if (rr.classify(a) != want) {
          std::printf("RowRanges<%d> mismatch %s c=%d a=%d valid=%d got %d want %d\n", M, tag, c, a, valid,
                      rr.classify(a), want);
          return 1;
        }
      }
    }
  }
  return 0;
}

static int check_key_ranges(long* n) {
  for (int S : {1, 31, 64, 97, 200, 513, 1024})
    for (int causal = 0; causal < 2; ++causal)
      for (int w : {0, 1, 5, 64, 129, 300})
        for (int d : {1, 2, 3})
          for (int blk : {0, 33, 128})
            for (int pre : {0, 40, 130, 2000}) {
              if (d > 1 && pre > 0) continue;
              const MaskSpec m = make_mask_spec(S, causal, w, d, blk, pre);
              char tag[96];
              std::snprintf(tag, sizeof tag, "S=%d c=%d w=%d d=%d blk=%d p=%d", S, causal, w, d, blk, pre);
              for (int r = 0; r < num_residues(m); ++r) {
                const MaskGeom g = residue_geom(m, r);
                if (g.S <= 0) continue;
                if (check_key_ranges_n<32>(g, n, tag) || check_key_ranges_n<64>(g, n, tag)) return 1;
                if (check_row_ranges_m<64>(g, n, tag) || check_row_ranges_m<128>(g, n, tag)) return 1;
              }
            }
  return 0;
}

int main() {
  const int bn = 64;
  long n_bits = 0, n_rows = 0;
  if (check_hidden_bits(&n_bits)) return 1;
  if (check_query_range(&n_rows)) return 1;
  long n_class = 0;
  if (check_key_ranges(&n_class)) return 1;
  long checked = 0, fast = 0, wide_all = 0;
  const int seqs[] = {1, 63, 64, 65, 200, 511, 700, 1024};
  const int windows[] = {0, 1, 5, 64, 129, 300};
  const int dils[] = {1, 2, 3};
  const int blocks[] = {0, 33, 128, 256};
  const int prefixes[] = {0, 40, 130};
  const int bmhs[] = {64, 128};  // rows per row block (2 or 4 wavefronts)
  for (int S : seqs)
    for (int causal = 0; causal < 2; ++causal)
      for (int w : windows)
        for (int d : dils)
          for (int blk : blocks)
            for (int pre : prefixes) {
              if (d > 1 && pre > 0) continue;
              const MaskSpec m = make_mask_spec(S, causal, w, d, blk, pre);
              for (int r = 0; r < num_residues(m); ++r) {
                const MaskGeom g = residue_geom(m, r);
                if (g.S <= 0) continue;
                for (int bmh : bmhs) {
                  const int nblk = (g.S + bmh - 1) / bmh;
                  for (int b0 = 0; b0 < nblk; ++b0)
                    for (int b1 : {b0, b0 + 1, nblk - 1 - b0, -1}) {
                      if (b1 >= nblk) continue;
                      // the workgroup-uniform WIDE span: WIDE in every wavefront
                      const TileSpan all = wide_range_all(g, b0 * bmh, (b1 >= 0 ? b1 : b0) * bmh, b1 >= 0, bmh / 32, bn);
                      const int n_pre_all = (g.prefix + bn - 1) / bn;
                      for (int t = imax32(all.lo, n_pre_all); t <= all.hi; ++t) {
                        const int c = bn * t, dd = c + bn - 1;
                        if (dd > g.S - 1) {
                          std::printf("WIDE span past the end S=%d t=%d\n", S, t);
                          return 1;
                        }
                        for (int wave = 0; wave < bmh / 32; ++wave) {
                          const int a0 = b0 * bmh + 32 * wave, a1 = (b1 >= 0 ? b1 : b0) * bmh + 32 * wave;
                          const int k0 = a0 < g.S ? classify_tile(g, a0, imin32(a0 + 31, g.S - 1), c, dd) : (int)TILE_EMPTY;
                          const int k1 = b1 >= 0 && a1 < g.S ? classify_tile(g, a1, imin32(a1 + 31, g.S - 1), c, dd)
                                                             : (int)TILE_EMPTY;
                          ++checked;
                          if (!(k0 == TILE_EMPTY && k1 == TILE_FULL)) {
                            std::printf("WIDE span mismatch S=%d c=%d w=%d d=%d blk=%d p=%d r=%d bmh=%d wave=%d t=%d k=%d,%d\n",
                                        S, causal, w, d, blk, pre, r, bmh, wave, t, k0, k1);
                            return 1;
                          }
                        }
                        ++wide_all;
                      }
                      for (int wave = 0; wave < bmh / 32; ++wave) {
                        const int a0 = b0 * bmh + 32 * wave, a1 = (b1 >= 0 ? b1 : b0) * bmh + 32 * wave;
                        const bool v0 = a0 < g.S, v1 = b1 >= 0 && a1 < g.S;
                        const int e0 = imin32(a0 + 31, g.S - 1), e1 = imin32(a1 + 31, g.S - 1);
                        const FastRanges fr = fast_ranges(g, a0, e0, v0, a1, e1, v1, bn);
                        const int n_pre = (g.prefix + bn - 1) / bn;
                        for (int t = n_pre; t <= g.S / bn + 1; ++t) {
                          const int c = bn * t, dd = c + bn - 1;
                          if (c > g.S - 1) break;
                          const int k0 = v0 ? classify_tile(g, a0, e0, c, dd) : (int)TILE_EMPTY;
                          const int k1 = v1 ? classify_tile(g, a1, e1, c, dd) : (int)TILE_EMPTY;
                          ++checked;
                          const bool in_p = t >= fr.pf_lo && t <= fr.pf_hi;
                          const bool in_w = t >= fr.wf_lo && t <= fr.wf_hi;
                          if (in_p && !in_w && !(k0 == TILE_FULL && k1 == TILE_FULL)) {
                            std::printf("PAIR mismatch S=%d c=%d w=%d d=%d blk=%d p=%d r=%d bmh=%d a0=%d a1=%d t=%d k=%d,%d\n",
                                        S, causal, w, d, blk, pre, r, bmh, a0, a1, t, k0, k1);
                            return 1;
                          }
                          if (in_w && !in_p && !(k0 == TILE_EMPTY && k1 == TILE_FULL)) {
                            std::printf("WIDE mismatch S=%d c=%d w=%d d=%d blk=%d p=%d r=%d bmh=%d a0=%d a1=%d t=%d k=%d,%d\n",
                                        S, causal, w, d, blk, pre, r, bmh, a0, a1, t, k0, k1);
                            return 1;
                          }
                          if (in_p && in_w) {
                            std::printf("overlapping fast ranges S=%d t=%d\n", S, t);
                            return 1;
                          }
                          fast += in_p || in_w;
                        }
                      }
                    }
                }
              }
            }
  std::printf("checked %ld band tiles, %ld on a fast path, %ld in a workgroup WIDE span, %ld mask bits, %ld query-range rows, "
              "%ld key-range classes\n",
              checked, fast, wide_all, n_bits, n_rows, n_class);
  return 0;
}
