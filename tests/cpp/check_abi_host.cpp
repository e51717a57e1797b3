// Host-side checks of the C ABI (include/chia_attn.h), built with
// AddressSanitizer and UndefinedBehaviorSanitizer on the host code by
// tests/test_sanitized_host.py.  Nothing here launches a kernel or needs a
// GPU: the checks cover the entry points that run on the host alone.
//   * status strings, versioning;
//   * argument validation of chia_attn_fwd, _fwd_lse, _bwd, _bwd_noalloc and
//     _fwd_fp8 (every path returns before any HIP call);
//   * chia_attn_plan's exact visible-pair count, chia_attn_tile_map's tile
//     classes and chia_attn_query_intervals' per-row intervals, against a
//     brute force written from the mask definition (extra_bench.py:41,56-61):
//     query i sees key j iff j < prefix or (band and same block and
//     (i - j) % dilation == 0).
// Exits non-zero on the first mismatch.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "chia_attn.h"

// The library's kernel selectors live in the kernel translation units, which
// this host-only build does not link: no call below reaches a launch.
namespace chia {
struct FwdParams;
struct BwdParams;
struct Fp8Params;
using KernelFn = void (*)(FwdParams);
using BwdKernelFn = void (*)(BwdParams);
using Fp8KernelFn = void (*)(Fp8Params);
struct BwdKernels {
  BwdKernelFn stats, dq, dkdv;
};
KernelFn select_kernel_d64(int, int, bool, bool) { return nullptr; }
KernelFn select_q1_kernel_d64(int, bool, bool, bool) { return nullptr; }
KernelFn select_kernel_d128(int) { return nullptr; }
KernelFn select_q1_kernel_d128(int, bool, bool, bool) { return nullptr; }
KernelFn select_q1_split_kernel_d128(int, bool, bool, bool) { return nullptr; }
BwdKernels select_bwd_kernels_d64(int, bool, bool) { return BwdKernels{nullptr, nullptr, nullptr}; }
BwdKernels select_bwd_kernels_d128(int, bool, bool) { return BwdKernels{nullptr, nullptr, nullptr}; }
Fp8KernelFn select_fp8_kernel(int, int, int, bool, bool) { return nullptr; }
}  // namespace chia

static int failures = 0;
static long conservative = 0;  // PARTIAL tiles that are in fact empty or full
#define CHECK(cond, ...)                                          \
  do {                                                            \
    if (!(cond)) {                                                \
      if (failures++ < 20) {                                      \
        std::printf("FAIL line %d: ", __LINE__);                  \
        std::printf(__VA_ARGS__);                                 \
        std::printf("\n");                                        \
      }                                                           \
    }                                                             \
  } while (0)

struct Mask {
  int S, causal, window, dil, block, prefix;
};

// The mask's definition, in original positions.
static bool visible(const Mask& m, long i, long j) {
  if (i < 0 || j < 0 || i >= m.S || j >= m.S) return false;
  if (j < m.prefix) return true;
  const long d = i - j;
  bool band = m.causal ? d >= 0 : true;
  if (m.window > 0) band = band && (m.causal ? d < m.window : (d < 0 ? -d : d) < m.window);
  const bool blk = m.block == 0 || i / m.block == j / m.block;
  return band && blk && d % m.dil == 0;
}

static chia_attn_args args_of(const Mask& m, int B = 1, int H = 1, int D = 64) {
  chia_attn_args a;
  std::memset(&a, 0, sizeof(a));
  a.struct_size = sizeof(a);
  a.norm = CHIA_ATTN_NORM_SOFTMAX;
  a.batch = B;
  a.heads = H;
  a.seqlen = m.S;
  a.head_dim = D;
  a.causal = m.causal;
  a.window = m.window;
  a.dilation = m.dil;
  a.block = m.block;
  a.prefix = m.prefix;
  a.scale = 0.125f;
  return a;
}

// Fake, aligned, never dereferenced device pointers for the validation paths.
static void fake_tensors(chia_attn_args* a) {
  a->q = (const void*)0x10000;
  a->k = (const void*)0x20000;
  a->v = (const void*)0x30000;
  a->o = (void*)0x40000;
  for (int64_t* st : {a->q_stride, a->k_stride, a->v_stride, a->o_stride}) {
    st[0] = a->heads * a->seqlen * a->head_dim;
    st[1] = a->seqlen * a->head_dim;
    st[2] = a->head_dim;
  }
}

static void check_mask(const Mask& m) {
  chia_attn_args a = args_of(m, 2, 3);
  chia_attn_plan_info info;
  CHECK(chia_attn_plan(&a, &info) == CHIA_ATTN_OK, "plan status");
  long pairs = 0;
  for (long i = 0; i < m.S; ++i)
    for (long j = 0; j < m.S; ++j) pairs += visible(m, i, j);
  CHECK(info.pairs_visible == 6 * pairs, "S%d c%d w%d d%d b%d p%d: plan pairs %lld, brute force %ld", m.S, m.causal,
        m.window, m.dil, m.block, m.prefix, (long long)info.pairs_visible, 6 * pairs);
  CHECK(info.wave_tiles_partial <= info.wave_tiles_visited, "partial tiles");
  const int R = m.dil < m.S ? m.dil : m.S;
  CHECK(info.residues == R, "residues %d vs %d", info.residues, R);
  for (int r = 0; r < R; ++r) {
    const int Sr = (m.S - r + m.dil - 1) / m.dil;  // sub-sequence i' -> r + dil i'
    auto vis = [&](long i2, long j2) { return visible(m, r + (long)m.dil * i2, r + (long)m.dil * j2); };
    // per-row intervals
    std::vector<int32_t> jlo(Sr), jhi(Sr);  // exact size: an overrun is an ASan report
    int32_t pre = -1;
    CHECK(chia_attn_query_intervals(&a, r, jlo.data(), jhi.data(), &pre, Sr) == CHIA_ATTN_OK, "intervals status");
    for (long i2 = 0; i2 < Sr; ++i2)
      for (long j2 = 0; j2 < Sr; ++j2) {
        const bool got = j2 < pre || (j2 >= jlo[i2] && j2 <= jhi[i2]);
        CHECK(got == vis(i2, j2), "interval r%d i'%ld j'%ld", r, i2, j2);
      }
    // tile classes for two block heights
    for (int rows : {32, 128}) {
      int32_t nqb = 0, nkt = 0;
      CHECK(chia_attn_tile_map(&a, r, rows, &nqb, &nkt, nullptr, 0) == CHIA_ATTN_OK, "tile map sizes");
      std::vector<int8_t> map((size_t)nqb * nkt);
      CHECK(chia_attn_tile_map(&a, r, rows, &nqb, &nkt, map.data(), (int64_t)map.size()) == CHIA_ATTN_OK, "tile map");
      for (int qb = 0; qb < nqb; ++qb)
        for (int kt = 0; kt < nkt; ++kt) {
          long seen = 0, all = 0;
          for (long i2 = (long)qb * rows; i2 < (long)(qb + 1) * rows && i2 < Sr; ++i2)
            for (long j2 = (long)kt * 64; j2 < (long)(kt + 1) * 64; ++j2) {
              ++all;
              seen += j2 < Sr && vis(i2, j2);
            }
          // EMPTY and FULL are exact claims; PARTIAL only means "apply the
          // mask" and may be conservative (a tile straddling the prefix end).
          const int got = map[(size_t)qb * nkt + kt];
          CHECK(got >= 0 && got <= 2, "tile class value %d", got);
          CHECK(got != 0 || seen == 0, "EMPTY tile with visible pairs r%d rows%d qb%d kt%d", r, rows, qb, kt);
          CHECK(got != 1 || seen == all, "FULL tile with hidden pairs r%d rows%d qb%d kt%d", r, rows, qb, kt);
          conservative += got == 2 && (seen == 0 || seen == all);
        }
    }
  }
}

// Planning at sizes whose pair counts overflow 32 bits, against closed forms:
// causal S(S+1)/2; causal window w: w(w+1)/2 + (S - w) w; block b (S a
// multiple of b): S b; prefix p, causal: p S + (S - p)(S - p + 1)/2.
static void check_large_plans() {
  const long S = 1 << 18, B = 64, H = 64, w = 256, b = 4096, p = 1024;
  struct Case {
    Mask m;
    long pairs;
  } cases[] = {
      {{(int)S, 1, 0, 1, 0, 0}, S * (S + 1) / 2},
      {{(int)S, 1, (int)w, 1, 0, 0}, w * (w + 1) / 2 + (S - w) * w},
      {{(int)S, 0, 0, 1, (int)b, 0}, S * b},
      {{(int)S, 1, 0, 1, 0, (int)p}, p * S + (S - p) * (S - p + 1) / 2},
  };
  for (const Case& c : cases) {
    chia_attn_args a = args_of(c.m, (int)B, (int)H);
    chia_attn_plan_info info;
    CHECK(chia_attn_plan(&a, &info) == CHIA_ATTN_OK, "large plan status");
    CHECK(info.pairs_visible == B * H * c.pairs, "large plan c%d w%d b%d p%d: %lld vs %ld", c.m.causal, c.m.window,
          c.m.block, c.m.prefix, (long long)info.pairs_visible, B * H * c.pairs);
    CHECK(info.wave_tiles_visited * 32 * 64 >= info.pairs_visible, "tiles cover the pairs");
  }
}

static void check_buffers() {
  chia_attn_args a = args_of(Mask{300, 1, 17, 3, 0, 0});
  int32_t nqb = 0, nkt = 0, pre = 0;
  CHECK(chia_attn_tile_map(&a, 0, 32, &nqb, &nkt, nullptr, 0) == CHIA_ATTN_OK, "tile map sizes");
  std::vector<int8_t> map((size_t)nqb * nkt - 1);
  CHECK(chia_attn_tile_map(&a, 0, 32, &nqb, &nkt, map.data(), (int64_t)map.size()) == CHIA_ATTN_ERR_SHAPE,
        "short tile map");
  CHECK(chia_attn_tile_map(&a, 3, 32, &nqb, &nkt, nullptr, 0) == CHIA_ATTN_ERR_MASK, "residue out of range");
  CHECK(chia_attn_tile_map(&a, 0, 0, &nqb, &nkt, nullptr, 0) == CHIA_ATTN_ERR_MASK, "zero rows");
  std::vector<int32_t> lo(99), hi(99);
  CHECK(chia_attn_query_intervals(&a, 0, lo.data(), hi.data(), &pre, 99) == CHIA_ATTN_ERR_SHAPE, "short intervals");
  CHECK(chia_attn_query_intervals(&a, -1, lo.data(), hi.data(), &pre, 99) == CHIA_ATTN_ERR_MASK, "negative residue");
  CHECK(chia_attn_plan(&a, nullptr) == CHIA_ATTN_ERR_NULL, "plan null");
}

static void check_validation() {
  Mask m{128, 1, 0, 1, 0, 0};
  chia_attn_args a = args_of(m, 1, 4);
  fake_tensors(&a);
  CHECK(chia_attn_fwd(nullptr, nullptr) == CHIA_ATTN_ERR_NULL, "null args");
  chia_attn_args b = a;
  b.struct_size = 8;
  CHECK(chia_attn_fwd(&b, nullptr) == CHIA_ATTN_ERR_STRUCT, "struct size");
  b = a;
  b.head_dim = 96;
  CHECK(chia_attn_fwd(&b, nullptr) == CHIA_ATTN_ERR_HEAD_DIM, "head dim");
  b = a;
  b.norm = 7;
  CHECK(chia_attn_fwd(&b, nullptr) == CHIA_ATTN_ERR_NORM, "norm");
  b = a;
  b.window = -1;
  CHECK(chia_attn_fwd(&b, nullptr) == CHIA_ATTN_ERR_MASK, "window");
  b = a;
  b.dilation = 2;
  b.prefix = 3;
  CHECK(chia_attn_fwd(&b, nullptr) == CHIA_ATTN_ERR_MASK, "prefix with dilation");
  b = a;
  b.scale = 0.f;
  CHECK(chia_attn_fwd(&b, nullptr) == CHIA_ATTN_ERR_SCALE, "scale");
  b = a;
  b.softcap = -1.f;
  CHECK(chia_attn_fwd(&b, nullptr) == CHIA_ATTN_ERR_SCALE, "softcap");
  b = a;
  b.q = (const void*)0x10008;
  CHECK(chia_attn_fwd(&b, nullptr) == CHIA_ATTN_ERR_ALIGN, "alignment");
  b = a;
  b.k_stride[2] = 68;
  CHECK(chia_attn_fwd(&b, nullptr) == CHIA_ATTN_ERR_ALIGN, "stride multiple of 8");
  b = a;
  b.kv_heads = 3;
  CHECK(chia_attn_fwd(&b, nullptr) == CHIA_ATTN_ERR_SHAPE, "kv heads");
  b = a;
  b.reserved[1] = 1;
  CHECK(chia_attn_fwd(&b, nullptr) == CHIA_ATTN_ERR_STRUCT, "reserved");
  b = a;
  b.batch = 0;
  CHECK(chia_attn_fwd(&b, nullptr) == CHIA_ATTN_ERR_SHAPE, "empty batch");
  CHECK(chia_attn_fwd_lse(&a, nullptr, nullptr) == CHIA_ATTN_ERR_NULL, "softmax lse required");

  // backward
  CHECK(chia_attn_bwd_workspace_size(&a) == 2 * 1 * 4 * 128 * 4, "workspace size");
  chia_attn_bwd_args w;
  std::memset(&w, 0, sizeof(w));
  w.struct_size = sizeof(w);
  w.fwd = &a;
  w.dout = (const void*)0x50000;
  w.dq = (void*)0x60000;
  w.dk = (void*)0x70000;
  w.dv = (void*)0x80000;
  for (int64_t* st : {w.dout_stride, w.dq_stride, w.dk_stride, w.dv_stride}) {
    st[0] = 4 * 128 * 64;
    st[1] = 128 * 64;
    st[2] = 64;
  }
  w.lse = (const float*)0x90000;
  CHECK(chia_attn_bwd(nullptr, nullptr) == CHIA_ATTN_ERR_NULL, "bwd null");
  CHECK(chia_attn_bwd(&w, nullptr) == CHIA_ATTN_ERR_WORKSPACE, "bwd needs a workspace");
  w.workspace = (void*)0xa0000;
  w.workspace_bytes = 8;
  CHECK(chia_attn_bwd(&w, nullptr) == CHIA_ATTN_ERR_WORKSPACE, "bwd workspace too small");
  chia_attn_bwd_args w2 = w;
  w2.reserved[3] = 1;
  CHECK(chia_attn_bwd(&w2, nullptr) == CHIA_ATTN_ERR_STRUCT, "bwd reserved");
  w2 = w;
  w2.dk = nullptr;
  CHECK(chia_attn_bwd_noalloc(&w2, nullptr) == CHIA_ATTN_ERR_NULL, "noalloc null output");
  // statistics beyond the static scratch are refused before any launch
  chia_attn_args big = args_of(Mask{8192, 1, 0, 1, 0, 0}, 16, 16);
  fake_tensors(&big);
  chia_attn_bwd_args wb = w;
  wb.fwd = &big;
  CHECK(chia_attn_bwd_workspace_size(&big) > (int64_t)CHIA_ATTN_NOALLOC_SCRATCH_BYTES, "big workspace");
  CHECK(chia_attn_bwd_noalloc(&wb, nullptr) == CHIA_ATTN_ERR_SCRATCH, "noalloc scratch limit");

  // FP8
  chia_attn_fp8_args f;
  std::memset(&f, 0, sizeof(f));
  f.struct_size = sizeof(f);
  f.attn = &a;
  f.q_descale = f.k_descale = f.v_descale = 1.f;
  CHECK(chia_attn_fwd_fp8(nullptr, nullptr) == CHIA_ATTN_ERR_NULL, "fp8 null");
  f.format = 2;
  CHECK(chia_attn_fwd_fp8(&f, nullptr) == CHIA_ATTN_ERR_STRUCT, "fp8 format");
  f.format = 0;
  f.v_descale = -1.f;
  CHECK(chia_attn_fwd_fp8(&f, nullptr) == CHIA_ATTN_ERR_SCALE, "fp8 descale");

  // status strings
  for (int st = -10; st <= 0; ++st) CHECK(std::strlen(chia_attn_status_string(st)) > 0, "status string %d", st);
  CHECK(std::strstr(chia_attn_status_string(-99), "unknown") != nullptr, "unknown status");
  CHECK(chia_attn_abi_version() == CHIA_ATTN_ABI_VERSION, "abi version");
}

int main() {
  check_validation();
  check_buffers();
  check_large_plans();
  int n = 0;
  for (int S : {1, 7, 64, 65, 130, 257, 300})
    for (int causal : {0, 1})
      for (int window : {0, 1, 17, 64, 400})
        for (int dil : {1, 2, 3})
          for (int block : {0, 32, 100})
            for (int prefix : {0, 5, 70}) {
              if (dil > 1 && prefix > 0) continue;  // rejected combination
              check_mask(Mask{S, causal, window, dil, block, prefix});
              ++n;
            }
  std::printf("%d masks checked, %d failures, %ld conservative PARTIAL tiles\n", n, failures, conservative);
  return failures ? 1 : 0;
}
