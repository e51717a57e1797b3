// Host model of the paired forward core's tile schedule
// (chia_proj_amd/csrc/attn_fwd_kernel.h: the DMA prologue, sync_step /
// issue_upto, the WIDE2 steps, the pipelined run and the main loop), checked
// for every workgroup of many masks, shapes and kernel kinds:
//   1. every wavefront of a workgroup passes the same barriers and issues the
//      same tiles after each (the loads of a tile are split over all of them);
//   2. a tile a wavefront reads after barrier b was issued, and the wait
//      before b (in-order vmcnt: all but the last `allowed` tiles issued have
//      landed) covers it in every wavefront;
//   3. a tile is issued into a stage only after the barrier that follows the
//      last read of the stage's previous tile, in every wavefront.
// The step decisions use the same mask.h functions as the kernel
// (tile_range_keys, fast_ranges, wide_range_all); the loop control is
// restated here and must follow the kernel's.  Built and run by
// tests/test_mask_fast_ranges.py; exits non-zero on the first violation.
// Run with an argument, it plants each of four mistakes in the model instead
// and exits non-zero unless every one of them is caught.
#include <cstdio>
#include <initializer_list>
#include <vector>

#include "mask.h"

using namespace chia;

namespace {

constexpr int BN = 64;

// A mistake planted in the model (0: none): 1 the DMA issuing one tile further
// ahead than the stages allow; 2 the pipelined kernels scheduled like the
// others (kFly = NS - 2 and oldest = it, forgetting the pending step's reads
// of the previous tile); 3 a vmcnt wait that leaves one of the step's own
// tiles in flight; 4 the WIDE2 decision from the wavefront's own range instead
// of the workgroup's.
int g_mistake = 0;

struct Kind {
  const char* name;
  int nw;     // wavefronts per workgroup
  bool pipe;  // the pipelined run (sigmoid / ReLU without a score modifier)
  bool rev;   // key tiles walked backwards (ALiBi softmax)
};

// One wavefront's trace: per barrier, the tiles issued after it; per read,
// (barrier interval, tile).
struct Trace {
  std::vector<std::vector<int>> issued;   // issued[b]: tiles issued right after barrier b
  std::vector<int> landed_below;          // landed_below[b]: every tile < this had landed at barrier b
  std::vector<std::pair<int, int>> reads; // (interval, tile)
  int prologue = 0;                       // tiles issued before the first barrier
};

struct Wg {
  MaskGeom g;
  int blk0, blk1, bmh;
};

Trace run_wave(const Kind& k, const Wg& w, int wave) {
  const int NW = k.nw, NS = NW == 4 ? 4 : 2, BMH = w.bmh;
  const bool wide2 = NW == 4 && !k.pipe;
  const int kFly = NS - (k.pipe && g_mistake != 2 ? 3 : 2), kIssue = wide2 ? 2 : 1;
  const MaskGeom& g = w.g;
  const int X = w.blk1 >= 0 ? w.blk1 : w.blk0;
  const TileRange tr =
      tile_range_keys(g, key_lo(g, w.blk0 * BMH), key_hi(g, imin32(X * BMH + BMH - 1, g.S - 1)), BN);
  const int ntiles = tr.n_pre + tr.n2;
  auto seq_tile = [&](int i) { return tile_at(tr, k.rev ? ntiles - 1 - i : i); };
  auto in_band = [&](int i) { return k.rev ? i < tr.n2 : i >= tr.n_pre; };
  const int r0 = w.blk0 * BMH + 32 * wave, r1 = X * BMH + 32 * wave;
  const bool v0 = r0 < g.S, v1 = w.blk1 >= 0 && r1 < g.S;
  const FastRanges fr = fast_ranges(g, r0, imin32(r0 + 31, g.S - 1), v0, r1, imin32(r1 + 31, g.S - 1), v1, BN);
  TileSpan w2{1, 0};
  if (wide2) w2 = wide_range_all(g, w.blk0 * BMH, X * BMH, w.blk1 >= 0, NW, BN);
  if (wide2 && g_mistake == 4) w2 = TileSpan{fr.wf_lo, fr.wf_hi};

  Trace t;
  int dma_next = 0;
  auto issue_upto = [&](int last, std::vector<int>& out) {
    last = imin32(last, ntiles - 1);
    for (int i = 0; i < kIssue; ++i)
      if (dma_next <= last) out.push_back(dma_next++);
  };
  auto sync_step = [&](int it, int n, int oldest) {
    const int inflight = dma_next - (it + n);
    int allowed = 0;  // tiles the vmcnt wait lets stay in flight
    if (kFly >= 2 && inflight >= 2) allowed = 2;
    else if (kFly >= 1 && inflight >= 1) allowed = 1;
    if (g_mistake == 3) allowed = inflight + 1;  // one of the step's own tiles left in flight
    t.landed_below.push_back(dma_next - allowed);
    t.issued.emplace_back();
    issue_upto(oldest + NS - 1 + (g_mistake == 1 ? 1 : 0), t.issued.back());
  };
  auto interval = [&]() { return (int)t.issued.size() - 1; };
  auto sync_tile = [&](int it) { sync_step(it, 1, k.pipe && g_mistake != 2 ? it - 1 : it); };
  for (int i = 0; i <= kFly && i < ntiles; ++i) ++t.prologue;
  dma_next = imin32(kFly + 1, ntiles);

  int ia = ntiles, ib = ntiles;
  if (k.pipe) {
    const int lo = imax32(fr.pf_lo, tr.start2), hi = imin32(fr.pf_hi, tr.start2 + tr.n2 - 1);
    if (lo <= hi) {
      ia = tr.n_pre + (lo - tr.start2);
      ib = tr.n_pre + (hi - tr.start2) + 1;
    }
  }
  for (int it = 0; it < ntiles; ++it) {
    if (k.pipe && it == ia) {
      // step (tile, key block): QK^T of n with the PV of the pending step
      sync_tile(ia);
      t.reads.push_back({interval(), ia});
      for (int j = ia + 1; j < ib; ++j) {
        sync_tile(j);
        t.reads.push_back({interval(), j - 1});  // pending step and deferred chunk: tile j - 1
        t.reads.push_back({interval(), j});
      }
      it = ib - 1;
      continue;
    }
    if (wide2) {
      const int tt = seq_tile(it);
      const bool two = k.rev ? (in_band(it) && in_band(it + 1) && tt - 1 >= w2.lo && tt <= w2.hi)
                             : (it >= tr.n_pre && it + 1 < ntiles && tt >= w2.lo && tt + 1 <= w2.hi);
      if (two) {
        sync_step(it, 2, it);
        t.reads.push_back({interval(), it});
        t.reads.push_back({interval(), it + 1});
        ++it;
        continue;
      }
    }
    sync_tile(it);
    t.reads.push_back({interval(), it});
  }
  if (dma_next != ntiles) t.prologue = -1;  // every tile issued (a read would fail below otherwise)
  return t;
}

// 0 when the workgroup's schedule is safe; prints the first violation.
bool g_quiet = false;

int check_wg(const Kind& k, const Wg& w, const char* what) {
  std::vector<Trace> tr;
  for (int wave = 0; wave < k.nw; ++wave) tr.push_back(run_wave(k, w, wave));
  const int NS = k.nw == 4 ? 4 : 2;
  for (int wave = 1; wave < k.nw; ++wave)
    if (tr[wave].issued != tr[0].issued || tr[wave].prologue != tr[0].prologue ||
        tr[wave].landed_below != tr[0].landed_below) {
      if (!g_quiet) std::printf("%s %s blk %d/%d: wavefront %d's barriers or loads differ from wavefront 0's\n", k.name, what,
                  w.blk0, w.blk1, wave);
      return 1;
    }
  // the interval in which each tile was issued (-1: the prologue)
  std::vector<int> issued_at;
  for (int i = 0; i < tr[0].prologue; ++i) issued_at.push_back(-1);
  for (int b = 0; b < (int)tr[0].issued.size(); ++b)
    for (int tile : tr[0].issued[b]) {
      if (tile != (int)issued_at.size()) {
        if (!g_quiet) std::printf("%s %s: tiles issued out of order\n", k.name, what);
        return 1;
      }
      issued_at.push_back(b);
    }
  if (tr[0].prologue < 0) {
    if (!g_quiet) std::printf("%s %s blk %d/%d: not every tile issued\n", k.name, what, w.blk0, w.blk1);
    return 1;
  }
  std::vector<int> last_read(issued_at.size(), -1);
  for (const Trace& t : tr)
    for (auto [b, tile] : t.reads) {
      if (tile < 0 || tile >= (int)issued_at.size() || issued_at[tile] >= b) {
        if (!g_quiet) std::printf("%s %s blk %d/%d: tile %d read after barrier %d before it was issued\n", k.name, what, w.blk0,
                    w.blk1, tile, b);
        return 1;
      }
      for (const Trace& u : tr)  // every wavefront's part has landed by barrier b
        if (!(tile < u.landed_below[b])) {
          if (!g_quiet) std::printf("%s %s blk %d/%d: tile %d read after barrier %d, not yet waited for\n", k.name, what, w.blk0,
                      w.blk1, tile, b);
          return 1;
        }
      last_read[tile] = imax32(last_read[tile], b);
    }
  for (int tile = NS; tile < (int)issued_at.size(); ++tile)
    if (!(last_read[tile - NS] < issued_at[tile])) {
      if (!g_quiet) std::printf("%s %s blk %d/%d: tile %d issued after barrier %d over tile %d, still read after barrier %d\n",
                  k.name, what, w.blk0, w.blk1, tile, issued_at[tile], tile - NS, last_read[tile - NS]);
      return 1;
    }
  return 0;
}

// Every workgroup of the sweep; the number of violating schedules (stops at the
// first when stop_first).
long sweep(long* wgs, bool stop_first) {
  const Kind kinds[] = {{"softmax-4w", 4, false, false}, {"alibi-softmax-4w", 4, false, true},
                        {"pipelined-4w", 4, true, false}, {"any-2w", 2, false, false},
                        {"alibi-softmax-2w", 2, false, true}};
  long bad = 0;
  char what[128];
  for (const Kind& k : kinds)
    for (int S : {1, 37, 64, 65, 200, 513, 1000, 2048})
      for (int causal = 0; causal < 2; ++causal)
        for (int win : {0, 1, 64, 129, 256, 700})
          for (int d : {1, 2, 3})
            for (int blk : {0, 33, 256})
              for (int pre : {0, 40, 300}) {
                if (d > 1 && pre > 0) continue;
                const MaskSpec m = make_mask_spec(S, causal, win, d, blk, pre);
                const int bmh = 32 * k.nw;
                for (int r = 0; r < num_residues(m); ++r) {
                  const MaskGeom g = residue_geom(m, r);
                  const int nblk = (g.S + bmh - 1) / bmh;
                  for (int zig = 0; zig < 2; ++zig)
                    for (int pr = 0; pr < (nblk + 1) / 2; ++pr) {
                      Wg w{g, 0, -1, bmh};
                      if (zig) {
                        w.blk0 = pr;
                        w.blk1 = nblk - 1 - pr;
                        if (w.blk1 < w.blk0) continue;
                        if (w.blk1 == w.blk0) w.blk1 = -1;
                      } else {
                        w.blk0 = 2 * pr;
                        w.blk1 = 2 * pr + 1;
                        if (w.blk0 >= nblk) continue;
                        if (w.blk1 >= nblk) w.blk1 = -1;
                      }
                      std::snprintf(what, sizeof what, "S=%d causal=%d window=%d dil=%d block=%d prefix=%d r=%d zig=%d",
                                    S, causal, win, d, blk, pre, r, zig);
                      ++*wgs;
                      if (check_wg(k, w, what)) {
                        ++bad;
                        if (stop_first) return bad;
                      }
                    }
                }
              }
  return bad;
}

}  // namespace

int main(int argc, char**) {
  long wgs = 0;
  if (argc > 1) {  // each planted mistake must be caught
    g_quiet = true;
    for (g_mistake = 1; g_mistake <= 4; ++g_mistake) {
      long n = 0;
      const long bad = sweep(&n, false);
      std::printf("planted mistake %d: %ld of %ld workgroup schedules violate\n", g_mistake, bad, n);
      if (bad == 0) return 1;
    }
    return 0;
  }
  if (sweep(&wgs, true)) return 1;
  std::printf("%ld workgroup schedules checked, 0 violations\n", wgs);
  return 0;
}
