// check_q1_split.cpp -- host restatement of the one-block core's loop control
// (attn_fwd_q1_kernel.h) with one or two groups per workgroup, checked for
// every zigzag pair of a sweep of masks and lengths:
//   * the two groups' step ranges cover the pair's steps exactly once, and
//     every block is computed whole by one group or split between the two
//     exactly where the kernel merges it;
//   * both groups pass the same number of workgroup barriers (steps, empty
//     steps, the merge's two), in the same roles;
//   * per group, the two-stage DMA: each step's tile was issued before its
//     barrier and waited for (vmcnt(0)), and a stage is refilled only after
//     the barrier that follows its last read;
//   * the merge buffer fits the workgroup's LDS.
// Build: g++ -std=c++17 -O2 -I chia_proj_amd/csrc tests/cpp/check_q1_split.cpp
#include <cstdio>
#include <vector>

#include "mask.h"

using namespace chia;

namespace {

constexpr int BN = 64, BM = 128, NS = 2;

struct Group {
  std::vector<char> bars;  // per barrier: 's' step, 'e' empty step, 'x' merge
  std::vector<int> steps;  // combined step indices computed, in order
  bool merges = false;     // computes part of the split block
};

int fails = 0;
int g_mistake = 0;  // > 0: a planted mistake the checks must catch
#define CHECK(c, ...)                 \
  do {                                \
    if (!(c)) {                       \
      if (fails++ < 10) {             \
        std::printf(__VA_ARGS__);     \
        std::printf("\n");            \
      }                               \
    }                                 \
  } while (0)

// One group's walk, following the kernel's statements.
Group walk(const MaskGeom& g, int blk0, int blk1, int NG, int grp, int* split_out) {
  const TileRange tr0 = tile_range(g, blk0 * BM, imin32(blk0 * BM + BM - 1, g.S - 1), BN);
  const int n0 = tr0.n_pre + tr0.n2;
  TileRange tr1{0, 0, 0};
  if (blk1 >= 0) tr1 = tile_range(g, blk1 * BM, imin32(blk1 * BM + BM - 1, g.S - 1), BN);
  const int nsteps = n0 + tr1.n_pre + tr1.n2;
  int M = NG == 2 ? (nsteps + 1) / 2 : nsteps;
  if (NG == 2 && blk1 >= 0 && M < n0) M = n0;
  const int s_lo = grp == 1 ? M + (g_mistake == 2) : 0, s_hi = grp == 1 ? nsteps : M;
  const int n_bar = imax32(M, nsteps - M);
  int split_pass = NG == 2 && M > 0 && M < nsteps ? (blk1 >= 0 ? (M > n0 ? 1 : -1) : 0) : -1;
  if (g_mistake == 4) split_pass = -1;
  *split_out = split_pass;

  Group G;
  // DMA model: issued[s] = barrier count at issue time (-1: prologue); stage of step s = s % NS
  std::vector<int> issued_at(nsteps + 1, -2), read_at_bar(nsteps + 1, -1);
  int dma_next = s_lo, nb = 0;
  for (; dma_next < s_lo + NS - 1 && dma_next < s_hi; ++dma_next) issued_at[dma_next] = -1;
  int step = s_lo;
  bool merged = false;
  for (int pass = 0; pass < 2; ++pass) {
    const int blk = pass == 0 ? blk0 : blk1;
    if (blk < 0) break;
    const int nt = pass == 0 ? n0 : tr1.n_pre + tr1.n2;
    const int base = pass == 0 ? 0 : n0;
    const int it_lo = imax32(s_lo - base, 0), it_hi = imin32(s_hi - base, nt);
    if (it_lo >= it_hi) continue;
    for (int it = it_lo; it < it_hi; ++it, ++step) {
      // vmcnt(0): every tile this group issued so far has landed
      G.bars.push_back('s');
      ++nb;
      CHECK(issued_at[step] != -2, "step %d computed but never issued", step);
      // refills stage dma_next % NS: its previous occupant (dma_next - NS) was
      // read in the interval before this barrier at the latest
      auto issue = [&](int s) {
        if (s - NS >= s_lo) CHECK(read_at_bar[s - NS] >= 0 && read_at_bar[s - NS] < nb, "stage of step %d refilled while read", s - NS);
        issued_at[s] = nb;
      };
      if (dma_next < s_hi) issue(dma_next++);
      if (g_mistake == 3 && dma_next < s_hi) issue(dma_next++);
      CHECK(issued_at[step] < nb, "step %d read after barrier %d but issued at %d", step, nb, issued_at[step]);
      read_at_bar[step] = nb;  // read in the interval after barrier nb
      CHECK(step == base + it, "step index drift");
      G.steps.push_back(step);
    }
    if (NG == 2 && pass == split_pass) {
      merged = true;
      G.merges = true;
      for (int k = s_hi - s_lo; k < n_bar && g_mistake != 1; ++k) G.bars.push_back('e');
      G.bars.push_back('x');
      G.bars.push_back('x');
      if (grp == 1) return G;
    }
  }
  if (NG == 2 && !merged)
    for (int k = s_hi - s_lo; k < n_bar; ++k) G.bars.push_back('e');
  CHECK(dma_next == s_hi, "group %d issued %d of its steps up to %d", grp, dma_next, s_hi);
  return G;
}

void check_pair(const MaskGeom& g, int blk0, int blk1, const char* what) {
  const TileRange tr0 = tile_range(g, blk0 * BM, imin32(blk0 * BM + BM - 1, g.S - 1), BN);
  const int n0 = tr0.n_pre + tr0.n2;
  int n1 = 0;
  if (blk1 >= 0) {
    const TileRange tr1 = tile_range(g, blk1 * BM, imin32(blk1 * BM + BM - 1, g.S - 1), BN);
    n1 = tr1.n_pre + tr1.n2;
  }
  const int nsteps = n0 + n1;
  int sp0, sp1;
  const Group a = walk(g, blk0, blk1, 2, 0, &sp0), b = walk(g, blk0, blk1, 2, 1, &sp1);
  CHECK(sp0 == sp1, "%s: split pass differs", what);
  CHECK(a.bars.size() == b.bars.size(), "%s: barrier counts %zu vs %zu", what, a.bars.size(), b.bars.size());
  for (size_t k = 0; k < a.bars.size() && k < b.bars.size(); ++k)
    CHECK((a.bars[k] == 'x') == (b.bars[k] == 'x'), "%s: barrier %zu is a merge barrier in one group only", what, k);
  // coverage: every step once, group 0's steps before group 1's
  std::vector<int> seen(nsteps, 0);
  for (int s : a.steps) ++seen[s];
  for (int s : b.steps) ++seen[s];
  for (int s = 0; s < nsteps; ++s) CHECK(seen[s] == 1, "%s: step %d computed %d times", what, s, seen[s]);
  if (!a.steps.empty() && !b.steps.empty()) CHECK(a.steps.back() < b.steps.front(), "%s: ranges interleave", what);
  // a block whose steps both groups computed is exactly the merged one
  for (int pass = 0; pass < 2; ++pass) {
    const int lo = pass == 0 ? 0 : n0, hi = pass == 0 ? n0 : nsteps;
    bool in_a = false, in_b = false;
    for (int s : a.steps) in_a |= s >= lo && s < hi;
    for (int s : b.steps) in_b |= s >= lo && s < hi;
    CHECK((in_a && in_b) == (sp0 == pass), "%s: block %d split between the groups %d, merged %d", what, pass,
          in_a && in_b, sp0 == pass);
  }
  CHECK(a.merges == b.merges, "%s: one group merges alone", what);
  // the single-group walk is unchanged: all steps in order
  int spx;
  const Group one = walk(g, blk0, blk1, 1, 0, &spx);
  CHECK((int)one.steps.size() == nsteps && (int)one.bars.size() == nsteps, "%s: one-group walk", what);
}

}  // namespace

long sweep() {
  long pairs = 0;
  char what[160];
  for (int S : {1, 64, 100, 128, 129, 255, 256, 300, 511, 512, 1000, 1024, 2048, 4096})
    for (int d : {1, 2, 4})
      for (int pre : {0, 40, 256, 1000}) {
        if (d > 1 && pre > 0) continue;
        const MaskSpec m = make_mask_spec(S, 1, 0, d, 0, pre);  // causal, no window: zigzag pairs
        for (int r = 0; r < num_residues(m); ++r) {
          const MaskGeom g = residue_geom(m, r);
          const int nblk = (g.S + BM - 1) / BM;
          for (int pr = 0; pr < (nblk + 1) / 2; ++pr) {
            int blk0 = pr, blk1 = nblk - 1 - pr;
            if (blk1 < blk0) continue;
            if (blk1 == blk0) blk1 = -1;
            std::snprintf(what, sizeof what, "S=%d dil=%d prefix=%d r=%d pair %d/%d", S, d, pre, r, blk0, blk1);
            check_pair(g, blk0, blk1, what);
            ++pairs;
          }
        }
      }
  return pairs;
}

int main(int argc, char**) {
  if (argc > 1) {  // each planted mistake must be caught
    for (g_mistake = 1; g_mistake <= 4; ++g_mistake) {
      fails = 0;
      const long n = sweep();
      std::printf("planted mistake %d: %d violations over %ld pairs\n", g_mistake, fails, n);
      if (fails == 0) return 1;
    }
    return 0;
  }
  const long pairs = sweep();
  // LDS: the merge buffer (4 wavefronts x 64 lanes x (16 DB + 2) floats) within NG x NS stages
  for (int D : {64, 128}) {
    const int DB = D / 32, stage = 2 * BN * 2 * D;
    CHECK(4 * 64 * (16 * DB + 2) * 4 <= 2 * NS * stage, "D=%d merge buffer exceeds the stages", D);
  }
  if (fails) {
    std::printf("%d violations\n", fails);
    return 1;
  }
  std::printf("%ld zigzag pairs checked with two groups, 0 violations\n", pairs);
  return 0;
}
