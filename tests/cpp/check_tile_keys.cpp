// check_tile_keys.cpp -- the stepped tile keys of the one-block core
// (attn_fwd_q1_kernel.h: the DMA's key of step s is the previous step's plus
// or minus one tile, computed in full only at the breaks seam0, n0 and seam1)
// against the full formula step_key0, restated here, over random tile ranges
// of one or two blocks, forward and backward walks, the rotation of a single
// block's band, and every group start (the two-group split starts a group
// mid-sequence).  The single-block form of the FP8 and dQ kernels (breaks at
// the first tile and the seam) is the case without block 1.  With an argument,
// each planted mistake in the break positions must be caught.
// Build: g++ -std=c++17 -O2 -I chia_proj_amd/csrc tests/cpp/check_tile_keys.cpp
#include <cstdio>
#include <random>

#include "mask.h"

using namespace chia;

namespace {

constexpr int BN = 64;
int g_mistake = 0;

struct Case {
  TileRange tr0, tr1;
  bool two;  // block 1 present
  bool rev;  // walk each block's tiles from the last to the first
};

// the kernel's step_key0
int full_key(const Case& c, int s) {
  const int n0 = c.tr0.n_pre + c.tr0.n2, n1 = c.tr1.n_pre + c.tr1.n2;
  const int rot0 = (!c.rev && !c.two && c.tr0.n_pre == 0 && n0 > 1) ? c.tr0.start2 % n0 : 0;
  const int a0 = c.tr0.start2;
  if (rot0 != 0 && s < n0) return (a0 + s - rot0 + (s < rot0 ? n0 : 0)) * BN;
  return (s < n0 ? tile_at(c.tr0, c.rev ? n0 - 1 - s : s) : tile_at(c.tr1, c.rev ? n1 - 1 - (s - n0) : s - n0)) * BN;
}

// the kernel's stepped keys for steps [s_lo, s_hi); returns the number of mismatches
int stepped(const Case& c, int s_lo, int s_hi) {
  const int n0 = c.tr0.n_pre + c.tr0.n2;
  const int rot0 = (!c.rev && !c.two && c.tr0.n_pre == 0 && n0 > 1) ? c.tr0.start2 % n0 : 0;
  const int dkey = c.rev ? -BN : BN;
  int seam0 = rot0 != 0 ? rot0 : (c.rev ? c.tr0.n2 : c.tr0.n_pre);
  int seam1 = n0 + (c.rev ? c.tr1.n2 : c.tr1.n_pre);
  if (g_mistake == 1) seam0 += 1;
  if (g_mistake == 2) seam1 = n0 + (c.rev ? c.tr1.n_pre : c.tr1.n2);
  auto next_break = [&](int s) {
    if (s < seam0) return seam0;
    if (s < n0) return n0;
    if (s < seam1) return seam1;
    return 0x7fffffff;
  };
  int bad = 0, key = 0, brk = 0;
  for (int s = s_lo; s < s_hi; ++s) {
    if (s == s_lo || s == brk) {
      key = full_key(c, s);
      brk = next_break(s);
    } else {
      key += dkey;
    }
    bad += key != full_key(c, s);
  }
  return bad;
}

}  // namespace

int main(int argc, char**) {
  std::mt19937 rng(20261202);
  auto uni = [&](int lo, int hi) { return std::uniform_int_distribution<int>(lo, hi)(rng); };
  const int planted = argc > 1 ? 2 : 0;
  for (int m = 0; m <= planted; ++m) {
    g_mistake = m;
    long steps = 0, bad = 0;
    for (int it = 0; it < 100000; ++it) {
      Case c;
      c.rev = uni(0, 4) < 2;
      c.two = uni(0, 1) == 1;
      c.tr0 = TileRange{uni(0, 5), uni(0, 40), uni(0, 12)};
      if (c.tr0.n_pre + c.tr0.n2 == 0) continue;
      if (c.tr0.n_pre > 0) c.tr0.start2 = imax32(c.tr0.start2, c.tr0.n_pre);
      c.tr1 = c.two ? TileRange{uni(0, 5), uni(0, 40), uni(0, 12)} : TileRange{0, 0, 0};
      if (c.two && c.tr1.n_pre > 0) c.tr1.start2 = imax32(c.tr1.start2, c.tr1.n_pre);
      const int ns = c.tr0.n_pre + c.tr0.n2 + c.tr1.n_pre + c.tr1.n2;
      const int s_lo = uni(0, ns), s_hi = uni(s_lo, ns);
      steps += s_hi - s_lo;
      bad += stepped(c, s_lo, s_hi);
    }
    if (m == 0) {
      std::printf("%ld steps, %ld stepped keys differ from step_key0\n", steps, bad);
      if (bad != 0) return 1;
    } else {
      std::printf("planted mistake %d: %ld of %ld keys differ\n", m, bad, steps);
      if (bad == 0) return 1;
    }
  }
  return 0;
}
