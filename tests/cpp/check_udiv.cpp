// Check of udiv / make_udiv (chia_proj_amd/csrc/mask.h) against plain integer
// division: every divisor 1..4096 and a spread of larger ones (powers of two
// and their neighbours, seqlen-sized values, random), each against dividends
// 0..2^14, the multiples of d and their neighbours, the top of the range and
// random values below 2^31.  Also floor_udiv / ceil_udiv against floor_div /
// ceil_div for negative dividends.  Built and run by
// tests/test_mask_fast_ranges.py; exits non-zero on the first mismatch.
#include <cstdint>
#include <cstdio>
#include <vector>

#include "mask.h"

using namespace chia;

static uint64_t rng = 0x9e3779b97f4a7c15ull;
static uint32_t next32() {
  rng ^= rng << 13;
  rng ^= rng >> 7;
  rng ^= rng << 17;
  return (uint32_t)(rng >> 11);
}

static int check(int32_t d, int32_t n) {
  const UDiv f = make_udiv(d);
  const int32_t got = udiv(n, f), want = n / d;
  if (got != want) {
    std::printf("udiv mismatch d=%d n=%d got=%d want=%d\n", d, n, got, want);
    return 1;
  }
  return 0;
}

int main() {
  std::vector<int32_t> divs;
  for (int32_t d = 1; d <= 4096; ++d) divs.push_back(d);
  for (int k = 12; k <= 30; ++k)
    for (int32_t e : {-1, 0, 1}) divs.push_back((int32_t)((1ll << k) + e));
  for (int32_t d : {3 * 4096, 5 * 4096 + 3, 100000, 999999, (1 << 28) - 1, 268435399}) divs.push_back(d);
  for (int i = 0; i < 2000; ++i) divs.push_back(1 + (int32_t)(next32() % ((1u << 28) - 1)));
  long n_checked = 0;
  auto run = [&](int32_t d, int64_t n) {
    if (n < 0 || n >= ((int64_t)1 << 31)) return true;
    ++n_checked;
    return check(d, (int32_t)n) == 0;
  };
  for (int32_t d : divs) {
    bool ok = true;
    for (int32_t n = 0; n < (1 << 14); ++n) ok = ok && run(d, n);
    for (int64_t k = 1; k * d < ((int64_t)1 << 31) && k < 4096; ++k)
      for (int64_t e : {-1, 0, 1}) ok = ok && run(d, k * d + e);
    for (int64_t n : {0x7fffffffll, 0x7ffffffell, 0x40000000ll, 0x3fffffffll}) ok = ok && run(d, n);
    for (int i = 0; i < 512; ++i) ok = ok && run(d, next32() & 0x7fffffff);
    if (!ok) return 1;
  }
  // signed floor / ceiling as the residue geometry uses them
  for (int32_t d = 1; d <= 64; ++d) {
    const UDiv f = make_udiv(d);
    for (int32_t a = -5000; a <= 5000; ++a) {
      if (floor_udiv(a, d, f) != floor_div(a, d) || ceil_udiv(a, d, f) != ceil_div(a, d)) {
        std::printf("floor/ceil mismatch d=%d a=%d\n", d, a);
        return 1;
      }
    }
  }
  std::printf("udiv checked %ld (divisor, dividend) pairs\n", n_checked);
  return 0;
}
