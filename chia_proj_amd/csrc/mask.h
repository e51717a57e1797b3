// mask.h -- visibility geometry shared by the host planner and the gfx950 kernel.
//
// Every mask of the reference's operator set (extra_bench.py:41,56-61) is, for
// one query row, a contiguous interval of visible keys plus a key prefix that
// every query sees:
//
//   visible(i, j) = (j < prefix) || (key_lo(i) <= j <= key_hi(i))
//
// Dilation ((i-j) % d == 0, extra_bench.py:56) is removed before that by
// re-indexing: rows with i % d == r form an independent problem over the
// sub-sequence i' = (i - r) / d, in which the remaining band / block / prefix
// constraints are again an interval plus a prefix.  key_lo and key_hi are
// non-decreasing in i', which is what makes the per-tile classification below
// exact for EMPTY and FULL (a tile is FULL only if every pair is visible and
// EMPTY only if none is).
#pragma once
#include <stdint.h>

#if defined(__HIPCC__) || defined(__HIP__)
#define CHIA_HD __host__ __device__ inline
#else
#define CHIA_HD inline
#endif

namespace chia {

constexpr int32_t kInf = 1 << 29;  // band sentinel; seqlen is limited to < 2^28

enum TileClass : int32_t { TILE_EMPTY = 0, TILE_FULL = 1, TILE_PARTIAL = 2 };

// Division of a non-negative 31-bit n by a fixed d >= 1 as one multiply-high,
// an add and a shift (Granlund & Montgomery, "Division by invariant integers
// using multiplication", PLDI 1994, the round-up multiplier): with
// l = ceil(log2 d) and m = floor(2^32 (2^l - d) / d) + 1 < 2^32,
// n / d = (mulhi(m, n) + n) >> l, exact for 0 <= n < 2^31 (the sum stays
// below 2^32).  The multiplier is computed on the host.
struct UDiv {
  uint32_t m;
  int32_t l;
};

CHIA_HD UDiv make_udiv(int32_t d) {  // d >= 1 (host side: one 64-bit division)
  int32_t l = 0;
  while (((int64_t)1 << l) < d) ++l;
  const uint64_t num = ((uint64_t)1 << 32) * (((uint64_t)1 << l) - (uint64_t)d);
  return UDiv{(uint32_t)(num / (uint64_t)d + 1), l};
}

CHIA_HD int32_t udiv(int32_t n, UDiv f) {  // 0 <= n < 2^31
#if defined(__HIP_DEVICE_COMPILE__)
  const uint32_t t = __umulhi(f.m, (uint32_t)n);
#else
  const uint32_t t = (uint32_t)(((uint64_t)f.m * (uint32_t)n) >> 32);
#endif
  return (int32_t)((t + (uint32_t)n) >> f.l);
}

// One residue class in sub-sequence coordinates.
struct MaskGeom {
  int32_t S;       // sub-sequence length
  int32_t lo, hi;  // band: lo <= i' - j' <= hi  (+-kInf = unbounded)
  int32_t prefix;  // keys j' < prefix are visible to every query
  int32_t blk;     // block size in ORIGINAL positions, 0 = off
  int32_t dil, r;  // original position = r + dil * sub position
  UDiv blk_div, dil_div;
};

CHIA_HD int32_t imax32(int32_t a, int32_t b) { return a > b ? a : b; }
CHIA_HD int32_t imin32(int32_t a, int32_t b) { return a < b ? a : b; }

CHIA_HD int32_t floor_div(int32_t a, int32_t b) {  // b > 0
  int32_t q = a / b;
  return (a % b != 0 && a < 0) ? q - 1 : q;
}
CHIA_HD int32_t ceil_div(int32_t a, int32_t b) {  // b > 0
  int32_t q = a / b;
  return (a % b != 0 && a > 0) ? q + 1 : q;
}

// First visible key of query i' (ignoring the prefix).
CHIA_HD int32_t key_lo(const MaskGeom& g, int32_t i) {
  int32_t v = (g.hi >= kInf) ? 0 : i - g.hi;
  if (g.blk > 0) {
    const int32_t io = g.r + g.dil * i;
    const int32_t bs = udiv(io, g.blk_div) * g.blk;  // first original position of the block
    v = imax32(v, bs <= g.r ? 0 : udiv(bs - g.r + g.dil - 1, g.dil_div));
  }
  return imax32(v, 0);
}

// Last visible key of query i' (ignoring the prefix).
CHIA_HD int32_t key_hi(const MaskGeom& g, int32_t i) {
  int32_t v = (g.lo <= -kInf) ? g.S - 1 : i - g.lo;
  if (g.blk > 0) {
    const int32_t io = g.r + g.dil * i;
    const int32_t be = udiv(io, g.blk_div) * g.blk + g.blk - 1;  // last original position
    v = imin32(v, udiv(be - g.r, g.dil_div));                     // be >= io >= r
  }
  return imin32(v, g.S - 1);
}

CHIA_HD bool visible(const MaskGeom& g, int32_t i, int32_t j) {
  if (j < 0 || j >= g.S || i < 0 || i >= g.S) return false;
  if (j < g.prefix) return true;
  return j >= key_lo(g, i) && j <= key_hi(g, i);
}

// Bits [a, b] of a 32-bit word (keys a..b counted from a block's first key),
// clipped to [0, 31]; 0 when the range misses the word or is empty.
CHIA_HD uint32_t key_bits(int32_t a, int32_t b) {
  const int32_t lo = a < 0 ? 0 : (a > 32 ? 32 : a);
  int32_t hi = b + 1 > 32 ? 32 : b + 1;
  hi = hi < lo ? lo : hi;
  return (uint32_t)(((uint64_t)1 << hi) - ((uint64_t)1 << lo));
}

// Keys jbase .. jbase + 31 that query i' does not see (also those past the
// end), as bits 0..31: the per-element mask of a partly visible key block.
CHIA_HD uint32_t hidden_bits(const MaskGeom& g, int32_t i, int32_t jbase) {
  return ~(key_bits(key_lo(g, i) - jbase, key_hi(g, i) - jbase) | key_bits(-jbase, g.prefix - 1 - jbase));
}

// Classify queries [a, b] (a <= b <= S-1) against keys [c, d] (c <= S-1; d
// may run past the end, those keys are treated as masked).
CHIA_HD int32_t classify_tile(const MaskGeom& g, int32_t a, int32_t b, int32_t c, int32_t d) {
  const bool tail = d > g.S - 1;
  if (!tail && d < g.prefix) return TILE_FULL;
  const int32_t ulo = key_lo(g, a), uhi = key_hi(g, b);  // hull of the rows' intervals
  if (ulo > uhi || c > uhi || d < ulo) return c < g.prefix ? TILE_PARTIAL : TILE_EMPTY;
  const int32_t ilo = key_lo(g, b), ihi = key_hi(g, a);  // common part of the intervals
  if (!tail && c >= ilo && d <= ihi) return TILE_FULL;
  return TILE_PARTIAL;
}

// classify_tile(g, a, b, c, c + N - 1) for one block of rows [a, b] and any
// key offset c, as range checks on c from bounds set once per block:
// FULL when the keys lie in the prefix, or in the rows' common interval
// [key_lo(b), key_hi(a)], and not past S - 1; otherwise PARTIAL when some key
// lies in the prefix or in the hull [key_lo(a), key_hi(b)]; otherwise EMPTY,
// and always when the block has no rows (valid false).  An empty range has
// the origin 2^30: c - origin then reads as an unsigned number above any span
// (and an empty prefix bound is -2^30, below any key).
template <int N>
struct KeyRanges {
  int32_t pfx, pf_hi, bf_lo, v_lo;
  uint32_t bf_span, v_span;
  CHIA_HD KeyRanges(const MaskGeom& g, bool valid, int32_t a, int32_t b) {
    constexpr int32_t kNone = 1 << 30;
    const int32_t ulo = key_lo(g, a), uhi = key_hi(g, b), ilo = key_lo(g, b), ihi = key_hi(g, a);
    pfx = valid ? g.prefix : -kNone;                        // c < pfx: the first key lies in the prefix
    pf_hi = valid ? imin32(g.prefix, g.S) - N : -kNone;     // c <= pf_hi: all N keys do, before S
    const int32_t bf_hi = imin32(ihi - (N - 1), g.S - N);
    const bool has_bf = valid && bf_hi >= ilo;
    bf_lo = has_bf ? ilo : kNone;
    bf_span = has_bf ? (uint32_t)(bf_hi - ilo) : 0u;
    const bool has_v = valid && ulo <= uhi;
    v_lo = has_v ? ulo - (N - 1) : kNone;
    v_span = has_v ? (uint32_t)(uhi - v_lo) : 0u;
  }
  CHIA_HD int32_t classify(int32_t c) const {
    if (c <= pf_hi || (uint32_t)(c - bf_lo) <= bf_span) return TILE_FULL;
    if (c < pfx || (uint32_t)(c - v_lo) <= v_span) return TILE_PARTIAL;
    return TILE_EMPTY;
  }
};

// Band key tiles (index t, keys [bn t, bn t + bn - 1], t >= the prefix tiles)
// whose classes for two query blocks [a0, b0], [a1, b1] (v0 / v1: the block
// has rows) are known without classify_tile: [pf_lo, pf_hi] where both blocks
// are FULL, [wf_lo, wf_hi] where block 0 is past its key hull (EMPTY) and
// block 1 is FULL.  Empty ranges have lo > hi.
struct FastRanges {
  int32_t pf_lo, pf_hi, wf_lo, wf_hi;
};

// The same from the blocks' interval ends: for block 0, ilo0 = key_lo(b0),
// ihi0 = key_hi(a0), ulo0 = key_lo(a0), uhi0 = key_hi(b0); for block 1,
// ilo1 = key_lo(b1), ihi1 = key_hi(a1).  S is the sub-sequence length.
CHIA_HD FastRanges fast_ranges_keys(int32_t S, int32_t ilo0, int32_t ihi0, int32_t ulo0, int32_t uhi0, bool v0,
                                    int32_t ilo1, int32_t ihi1, bool v1, int32_t bn) {
  FastRanges r{1, 0, 1, 0};
  // FULL band tiles of a block: c >= key_lo(b), d <= key_hi(a), d <= S - 1
  const bool f0 = v0 && ilo0 <= ihi0, f1 = v1 && ilo1 <= ihi1;
  const int32_t lo0 = ceil_div(ilo0, bn), hi0 = imin32(floor_div(ihi0 + 1, bn), S / bn) - 1;
  const int32_t lo1 = ceil_div(ilo1, bn), hi1 = imin32(floor_div(ihi1 + 1, bn), S / bn) - 1;
  if (f0 && f1) {
    r.pf_lo = imax32(lo0, lo1);
    r.pf_hi = imin32(hi0, hi1);
  }
  if (f1) {
    // block 0 sees no key after its hull end key_hi(b0)
    const int32_t after0 = (v0 && ulo0 <= uhi0) ? uhi0 / bn + 1 : 0;
    r.wf_lo = imax32(lo1, after0);
    r.wf_hi = hi1;
  }
  return r;
}

CHIA_HD FastRanges fast_ranges(const MaskGeom& g, int32_t a0, int32_t b0, bool v0, int32_t a1, int32_t b1, bool v1,
                               int32_t bn) {
  return fast_ranges_keys(g.S, key_lo(g, b0), key_hi(g, a0), key_lo(g, a0), key_hi(g, b0), v0, key_lo(g, b1),
                          key_hi(g, a1), v1, bn);
}

// Band tiles in the WIDE range of every wavefront of a workgroup: wavefront w
// holds query blocks [r0 + 32 w, +32) and, when has1, [r1 + 32 w, +32).  A
// step that decides the workgroup's barrier schedule may only use this
// intersection, not one wavefront's own range.  Empty when lo > hi.
struct TileSpan {
  int32_t lo, hi;
};

CHIA_HD TileSpan wide_range_all(const MaskGeom& g, int32_t r0, int32_t r1, bool has1, int32_t nw, int32_t bn) {
  TileSpan s{0, 0x7fffffff};
  for (int32_t w = 0; w < nw; ++w) {
    const int32_t a0 = r0 + 32 * w, a1 = r1 + 32 * w;
    const FastRanges f = fast_ranges(g, a0, imin32(a0 + 31, g.S - 1), a0 < g.S, a1, imin32(a1 + 31, g.S - 1),
                                     has1 && a1 < g.S, bn);
    s.lo = imax32(s.lo, f.wf_lo);
    s.hi = imin32(s.hi, f.wf_hi);
  }
  return s;
}

// Queries (sub-sequence rows) that may see a key of [j0, j1]: every row when
// the block holds a prefix key, else the rows whose interval reaches j0
// (key_hi non-decreasing: a suffix) and starts by j1 (key_lo non-decreasing:
// a prefix).  A superset of the rows that see the block: rows inside whose
// interval misses it are classified EMPTY or masked.  Empty when lo > hi.
struct RowSpan {
  int32_t lo, hi;
};

CHIA_HD RowSpan query_range(const MaskGeom& g, int32_t j0, int32_t j1) {
  if (j0 < g.prefix) return RowSpan{0, g.S - 1};
  int32_t lo = 0, hi = g.S;  // first row with key_hi >= j0
  while (lo < hi) {
    const int32_t mid = (lo + hi) >> 1;
    if (key_hi(g, mid) >= j0) hi = mid;
    else lo = mid + 1;
  }
  const int32_t first = lo;
  lo = 0;
  hi = g.S;  // first row with key_lo > j1
  while (lo < hi) {
    const int32_t mid = (lo + hi) >> 1;
    if (key_lo(g, mid) > j1) hi = mid;
    else lo = mid + 1;
  }
  return RowSpan{first, lo - 1};
}

// classify_tile(g, a, min(a + M - 1, S - 1), c, d) for fixed keys [c, d]
// (c <= S - 1) and any row tile start a (0 <= a <= S - 1), from two row
// spans found once: the rows that see some key of [c, d] (query_range(c, d):
// key_hi(i) >= c and key_lo(i) <= d, or every row when c is in the prefix)
// and those that see all of them (query_range(d, c): key_hi(i) >= d and
// key_lo(i) <= c, or every row when d is in the prefix; none when d runs past
// S - 1).  FULL when the tile lies inside the second span, PARTIAL when it
// meets the first, EMPTY otherwise and for keys without a wavefront
// (valid false).  Exact because key_lo and key_hi are non-decreasing and
// every row sees its own key (key_lo(i) <= i <= key_hi(i)).
template <int M>
struct RowRanges {
  int32_t f_lo, f_hi, v_lo, v_hi, last;
  CHIA_HD RowRanges(const MaskGeom& g, bool valid, int32_t c, int32_t d) {
    constexpr int32_t kNone = 1 << 30;  // an empty span: no tile reaches it
    last = g.S - 1;
    const RowSpan v = valid ? query_range(g, c, d) : RowSpan{kNone, -kNone};
    const RowSpan f = valid && d <= g.S - 1 ? query_range(g, d, c) : RowSpan{kNone, -kNone};
    v_lo = v.lo;
    v_hi = v.hi;
    f_lo = f.lo;
    f_hi = f.hi;
  }
  CHIA_HD int32_t classify(int32_t a) const {
    const int32_t b = imin32(a + M - 1, last);
    if (a >= f_lo && b <= f_hi) return TILE_FULL;
    if (b >= v_lo && a <= v_hi) return TILE_PARTIAL;
    return TILE_EMPTY;
  }
};

// KV tiles of width bn that queries [a, b] may touch: [0, n_pre) followed by
// [start2, start2 + n2).
struct TileRange {
  int32_t n_pre, start2, n2;
};

// The same from the hull ends ulo = key_lo(g, a), uhi = key_hi(g, b).
CHIA_HD TileRange tile_range_keys(const MaskGeom& g, int32_t ulo, int32_t uhi, int32_t bn) {
  TileRange t;
  t.n_pre = (g.prefix + bn - 1) / bn;
  t.start2 = t.n_pre;
  t.n2 = 0;
  if (ulo <= uhi) {
    const int32_t t0 = ulo / bn, t1 = uhi / bn;
    t.start2 = imax32(t0, t.n_pre);
    t.n2 = imax32(0, t1 - t.start2 + 1);
  }
  return t;
}

CHIA_HD TileRange tile_range(const MaskGeom& g, int32_t a, int32_t b, int32_t bn) {
  return tile_range_keys(g, key_lo(g, a), key_hi(g, b), bn);
}

CHIA_HD int32_t tile_at(const TileRange& t, int32_t k) {
  return k < t.n_pre ? k : t.start2 + (k - t.n_pre);
}

// Host-side parameters of the whole problem (original coordinates).
struct MaskSpec {
  int32_t S;
  int32_t lo, hi;  // band in original units
  int32_t blk, prefix, dil;
  UDiv blk_div, dil_div;  // dividers by blk (when > 0) and dil
};

CHIA_HD MaskSpec make_mask_spec(int32_t S, int32_t causal, int32_t window, int32_t dilation,
                                int32_t block, int32_t prefix) {
  MaskSpec m;
  m.S = S;
  if (causal) {
    m.lo = 0;
    m.hi = window > 0 ? window - 1 : kInf;
  } else if (window > 0) {
    m.lo = -(window - 1);
    m.hi = window - 1;
  } else {
    m.lo = -kInf;
    m.hi = kInf;
  }
  m.blk = block;
  m.prefix = prefix;
  m.dil = dilation < 1 ? 1 : dilation;
  m.blk_div = make_udiv(block > 0 ? block : 1);
  m.dil_div = make_udiv(m.dil);
  return m;
}

CHIA_HD int32_t num_residues(const MaskSpec& m) { return imin32(m.dil, m.S); }

// Floor and ceiling of a / d for |a| < 2^30 with the divider of d.
CHIA_HD int32_t floor_udiv(int32_t a, int32_t d, UDiv f) { return a >= 0 ? udiv(a, f) : -udiv(-a + d - 1, f); }
CHIA_HD int32_t ceil_udiv(int32_t a, int32_t d, UDiv f) { return a >= 0 ? udiv(a + d - 1, f) : -udiv(-a, f); }

CHIA_HD MaskGeom residue_geom(const MaskSpec& m, int32_t r) {
  MaskGeom g;
  g.dil = m.dil;
  g.r = r;
  g.S = r < m.S ? udiv(m.S - r + m.dil - 1, m.dil_div) : 0;
  g.lo = m.lo <= -kInf ? -kInf : ceil_udiv(m.lo, m.dil, m.dil_div);
  g.hi = m.hi >= kInf ? kInf : floor_udiv(m.hi, m.dil, m.dil_div);
  g.blk = m.blk;
  g.blk_div = m.blk_div;
  g.dil_div = m.dil_div;
  const int32_t p = m.prefix > r ? udiv(m.prefix - r + m.dil - 1, m.dil_div) : 0;
  g.prefix = imin32(p, g.S);
  return g;
}

}  // namespace chia
