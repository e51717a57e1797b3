/*
 * chia_attn.h -- C ABI of the MI355X (gfx950) attention-variant forward library.
 *
 * One forward-attention core serves all ten variants of the reference's
 * operator set (sliding-window, local, dilated, block-diagonal, prefix-LM,
 * ALiBi, Gemma-2 softcap, per-head temperature, ReLU and sigmoid attention).
 * A variant is a combination of three independent parts of the argument
 * struct: a mask (causal / window / dilation / block / prefix), a score
 * modifier (scale, per-head scale, ALiBi slopes, softcap) and a normaliser
 * (softmax, sigmoid or ReLU).
 *
 * Every entry point takes plain pointers and sizes.  Tensors are bf16 device
 * buffers laid out [batch, heads, seqlen, head_dim] with arbitrary batch/head/
 * seq strides (in elements) and a unit head_dim stride.  The caller allocates
 * q, k, v, o and the per-head vectors; the library's only device memory is the
 * static scratch array of chia_attn_bwd_noalloc.
 *
 * Reference interface replaced (JoshiP-commits/CHIA_proj):
 *   kernels_gemini31propre_0018/<op>_BEST.py::launch_kernel(q, k, v) -> o
 *   (e.g. bias_sliding_window_BEST.py:87-108), whose semantics are the eager
 *   closures of extra_bench.py:32-62 and sigmoid_fix.py:34-40.
 */
#ifndef CHIA_ATTN_H
#define CHIA_ATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CHIA_ATTN_ABI_VERSION 4 /* 2: kv_heads (GQA / MQA); 3: cu_seqlens (packed sequences);
                                   4: chia_attn_bwd_noalloc and status -10, plan units per core
                                      (block_n is 32 keys on the one-block core, 64 on the paired core) */

/* Normaliser applied to the (modified, masked) scores.
 *   SOFTMAX: p = softmax_j(s) over visible keys   (extra_bench.py:42)
 *   SIGMOID: p = sigmoid(s + bias) * visible       (sigmoid_fix.py:37-39)
 *   RELU:    p = relu(s) * visible                 (extra_bench.py:44)
 * SIGMOID and RELU outputs are multiplied by post_scale. */
enum chia_attn_norm {
  CHIA_ATTN_NORM_SOFTMAX = 0,
  CHIA_ATTN_NORM_SIGMOID = 1,
  CHIA_ATTN_NORM_RELU = 2
};

/* Status codes.  0 is success; negative values are argument errors found on
 * the host before any launch; positive values are hipError_t codes returned
 * by the HIP runtime. */
enum chia_attn_status {
  CHIA_ATTN_OK = 0,
  CHIA_ATTN_ERR_NULL = -1,          /* NULL args, tensor or required pointer */
  CHIA_ATTN_ERR_SHAPE = -2,         /* batch/heads/seqlen < 1 or too large, a K/V seq
                                        stride < 0 or >= 2^25 / dilation elements, or
                                        kv_heads < 0 or not dividing heads              */
  CHIA_ATTN_ERR_HEAD_DIM = -3,      /* head_dim not in {64, 128}            */
  CHIA_ATTN_ERR_MASK = -4,          /* negative window/block/prefix, dilation < 1,
                                       or prefix > 0 with dilation > 1 */
  CHIA_ATTN_ERR_SCALE = -5,         /* scale <= 0, non-finite, softcap < 0  */
  CHIA_ATTN_ERR_NORM = -6,          /* unknown normaliser                   */
  CHIA_ATTN_ERR_ALIGN = -7,         /* pointer/stride not 16-byte aligned   */
  CHIA_ATTN_ERR_STRUCT = -8,        /* struct_size does not match this ABI  */
  CHIA_ATTN_ERR_WORKSPACE = -9,     /* backward workspace NULL or too small */
  CHIA_ATTN_ERR_SCRATCH = -10       /* chia_attn_bwd_noalloc: statistics exceed the static scratch */
};

typedef struct chia_attn_args {
  uint32_t struct_size;   /* sizeof(chia_attn_args) */
  uint32_t norm;          /* enum chia_attn_norm */

  const void* q;          /* bf16 [B, H, S, D] */
  const void* k;          /* bf16 [B, H_kv, S, D] (H_kv = kv_heads, or H) */
  const void* v;          /* bf16 [B, H_kv, S, D] */
  void* o;                /* bf16 [B, H, S, D], written */

  int64_t batch, heads, seqlen, head_dim;
  int64_t q_stride[3];    /* batch, head, seq strides in elements */
  int64_t k_stride[3];
  int64_t v_stride[3];
  int64_t o_stride[3];

  /* Mask.  Query i sees key j iff
   *   (j < prefix)  OR  (band(i,j) AND same_block(i,j) AND (i-j) % dilation == 0)
   * band: causal && window>0 : 0 <= i-j < window     (extra_bench.py:61)
   *       causal && window==0: 0 <= i-j              (extra_bench.py:41)
   *       !causal && window>0: |i-j| < window        (extra_bench.py:57)
   *       !causal && window==0: always
   * same_block: block==0 or i/block == j/block       (extra_bench.py:58)
   * prefix: prefix-LM keys visible to every query    (extra_bench.py:59)
   * prefix > 0 cannot be combined with dilation > 1. */
  int32_t causal;
  int32_t window;
  int32_t dilation;       /* >= 1; 1 = no dilation  (extra_bench.py:56) */
  int32_t block;          /* >= 0 */
  int32_t prefix;         /* >= 0 */

  /* Score s_ij = (q_i . k_j) * scale * head_scale[h] + slope[h] * (j - i),
   * then s = softcap * tanh(s / softcap) when softcap > 0. */
  float scale;                /* > 0, reference 1/sqrt(D) (extra_bench.py:33) */
  float softcap;              /* 0 = off (extra_bench.py:60) */
  float bias;                 /* SIGMOID: added before the sigmoid */
  float post_scale;           /* SIGMOID/RELU: multiplies p */
  const float* head_scale;    /* device float[heads], each > 0, or NULL (extra_bench.py:35,54) */
  const float* alibi_slopes;  /* device float[heads] or NULL (extra_bench.py:36,47-50) */

  /* Grouped-query / multi-query attention: K and V have kv_heads heads and
   * query head h reads K/V head h / (heads / kv_heads).  0 = heads (one K/V
   * head per query head).  heads % kv_heads must be 0.  The reference's
   * kernels take K and V of q's shape only; this generalises them. */
  int32_t kv_heads;
  int32_t reserved0;          /* must be zero */

  /* Variable-length batches (packed sequences).  NULL: every sequence has
   * seqlen tokens and the tensors are [B, H, S, D] as above.  Otherwise a
   * device int32[batch + 1] with cu_seqlens[0] = 0, non-decreasing: sequence b
   * is tokens [cu_seqlens[b], cu_seqlens[b + 1]) of packed tensors q, o
   * [T, H, D] and k, v [T, H_kv, D]; the batch strides (stride[0]) are ignored
   * and stride[2] steps one token.  seqlen must be >= every sequence's length
   * (rows beyond seqlen are not computed).  Masks and ALiBi positions count
   * from each sequence's first token.  The values are read by the GPU and not
   * checked: the caller guarantees them (the Python layer checks a host copy).
   * No counterpart in the reference, whose kernels take one fixed shape. */
  const int32_t* cu_seqlens;
  /* With cu_seqlens: NULL, or a device int32[batch] permutation of 0..batch-1,
   * the order in which the sequences' work is dispatched.  Longest first keeps
   * the longest sequences off the end of the launch (the Python layer passes
   * it).  Ignored without cu_seqlens; not checked on the GPU. */
  const int32_t* seq_order;
  int32_t reserved[2];        /* must be zero */
} chia_attn_args;

/* Launch one forward attention on `stream` (a hipStream_t; NULL = default
 * stream).  Asynchronous: returns after the launch is queued.  Replaces
 * launch_kernel(q, k, v) of kernels_gemini31propre_0018/<op>_BEST.py
 * (e.g. bias_sliding_window_BEST.py:87-108). */
int chia_attn_fwd(const chia_attn_args* args, void* stream);

/* chia_attn_fwd that also writes, for a SOFTMAX normaliser, the log-sum-exp of
 * each row's modified, masked scores: lse[(b * H + h) * S + i] (packed
 * sequences: lse[t * H + h] for token t) = log(sum_j visible exp(s_ij)), fp32,
 * -inf for a row that sees no key -- the
 * statistic chia_attn_bwd needs.  lse must be non-NULL (4-byte aligned) for
 * SOFTMAX and is ignored for SIGMOID / RELU.  No counterpart in the reference,
 * whose kernels are forward-only (README.md:223); this is the training
 * extension's forward. */
int chia_attn_fwd_lse(const chia_attn_args* args, float* lse, void* stream);

/* Backward of the forward `fwd` describes: given o, lse (SOFTMAX) and
 * dout = dL/do, writes dq = dL/dq [B, H, S, D] and dk, dv = dL/dk, dL/dv
 * [B, H_kv, S, D] (bf16; with kv_heads < heads, each K/V head's gradient is
 * the sum over its query heads).  head_scale and alibi_slopes are constants
 * (no gradient).  The gradients are those of the exact (unrounded) forward
 * with the probabilities recomputed from lse.  No counterpart in the
 * reference (forward-only, README.md:223). */
typedef struct chia_attn_bwd_args {
  uint32_t struct_size;       /* sizeof(chia_attn_bwd_args) */
  uint32_t reserved0;         /* must be zero */
  const chia_attn_args* fwd;  /* the forward's arguments: q, k, v, o and every parameter */
  const void* dout;           /* bf16 [B, H, S, D] */
  void* dq;                   /* bf16 [B, H, S, D], written */
  void* dk;                   /* bf16 [B, H_kv, S, D], written */
  void* dv;                   /* bf16 [B, H_kv, S, D], written */
  int64_t dout_stride[3];     /* batch, head, seq strides in elements */
  int64_t dq_stride[3];
  int64_t dk_stride[3];
  int64_t dv_stride[3];
  const float* lse;           /* SOFTMAX: [B, H, S] from chia_attn_fwd_lse; else ignored */
  void* workspace;            /* device memory of chia_attn_bwd_workspace_size bytes */
  int64_t workspace_bytes;
  int32_t reserved[8];        /* must be zero */
} chia_attn_bwd_args;

/* Bytes of workspace chia_attn_bwd needs for `fwd` (fp32 row statistics for
 * SOFTMAX, 0 otherwise); negative: an argument error. */
int64_t chia_attn_bwd_workspace_size(const chia_attn_args* fwd);

/* Launch the backward on `stream` (asynchronous; the caller keeps every
 * buffer alive until it completes).  Status codes as chia_attn_fwd. */
int chia_attn_bwd(const chia_attn_bwd_args* args, void* stream);

/* chia_attn_bwd that allocates nothing.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving or training loops, harnesses that forbid hipMalloc).
 * The row statistics that chia_attn_bwd keeps in the caller's workspace go to a
 * static device array of CHIA_ATTN_NOALLOC_SCRATCH_BYTES per GPU instead (held
 * by each GPU the library runs on until the process ends); the workspace and
 * workspace_bytes fields are ignored.  A problem whose statistics
 * (chia_attn_bwd_workspace_size) exceed that size returns
 * CHIA_ATTN_ERR_SCRATCH before any launch.  Call it with the device of
 * `stream` current.  Every call on one GPU shares that GPU's array: calls that
 * overlap in time on one GPU (other streams, other host threads) race and must
 * be serialised by the caller.  Nothing in the array needs clearing between
 * calls: each call writes the statistics of every row it has before any
 * kernel reads them, and the padding rows of a last partial tile, which are
 * read, never reach a result.  Results are those of chia_attn_bwd bit for bit
 * (the same kernels). */
#define CHIA_ATTN_NOALLOC_SCRATCH_BYTES (8 << 20)
int chia_attn_bwd_noalloc(const chia_attn_bwd_args* args, void* stream);

/* FP8 forward.  `attn` describes the call as for chia_attn_fwd, with q, k, v
 * pointing at float8 data of one format (`format`: OCP e4m3fn -- 4 exponent
 * bits, bias 7, max 448 -- or OCP e5m2 -- 5 exponent bits, bias 15, max
 * 57344; strides in elements = bytes, multiples of 16; 16-byte aligned) and o
 * at bf16 [B, H, S, D].  Real values are stored values times the descales.
 * Both products run on the gfx950 FP8 matrix path (twice the bf16 rate): the
 * weights are rounded to e4m3 after scaling by 2^8 (for either input format),
 * the accumulation is fp32; ReLU weights above 448 saturate.  Packed
 * sequences (cu_seqlens, seq_order) work as for chia_attn_fwd.  No
 * counterpart in the reference, whose kernels are bf16 only. */
#define CHIA_ATTN_FP8_E4M3 0u
#define CHIA_ATTN_FP8_E5M2 1u
typedef struct chia_attn_fp8_args {
  uint32_t struct_size;        /* sizeof(chia_attn_fp8_args) */
  uint32_t format;             /* CHIA_ATTN_FP8_E4M3 or CHIA_ATTN_FP8_E5M2: q, k and v */
  const chia_attn_args* attn;  /* shapes, strides, mask, score, normaliser; q, k, v fp8; o bf16 */
  float q_descale, k_descale, v_descale;  /* > 0, finite */
  int32_t reserved[5];         /* must be zero */
} chia_attn_fp8_args;

int chia_attn_fwd_fp8(const chia_attn_fp8_args* args, void* stream);

/* Host-only schedule statistics for `args` (no GPU call).  Used by the
 * benchmark's FLOP accounting; the reference has no counterpart (its timer,
 * extra_bench.py:8-22, counts latency only). */
typedef struct chia_attn_plan_info {
  int32_t block_m;          /* query rows a workgroup computes per KV tile: two row blocks
                               (paired core), one (head_dim 128 one-block core) */
  int32_t block_n;          /* keys per computed step: the 64-key KV tile (paired core) or
                               its 32-key halves (one-block core); tile counts below use it */
  int32_t wave_m;           /* rows of one computed sub-tile (32) */
  int32_t waves;            /* wavefronts per workgroup */
  int64_t workgroups;       /* grid size */
  int64_t tiles_total;      /* (workgroup step, block_n keys) pairs of the dense grid */
  int64_t tiles_visited;    /* (workgroup step, block_n keys) pairs loaded into LDS */
  int64_t wave_tiles_visited; /* (32-row block, block_n keys) pairs computed (wave_m x block_n) */
  int64_t wave_tiles_partial; /* of which need the per-element mask */
  int64_t pairs_visible;    /* exact number of visible (i, j) pairs over B*H */
  int32_t residues;         /* dilation classes the problem splits into */
  int32_t reserved[7];
} chia_attn_plan_info;

int chia_attn_plan(const chia_attn_args* args, chia_attn_plan_info* out);

/* Host-only tile map for one residue class: out[qb * n_kt + kt] is
 * 0 = empty, 1 = full, 2 = partial for query block qb (rows_per_block rows)
 * and key tile kt (block_n keys), classified with the same functions the
 * kernel uses.  n_qb/n_kt are returned through the pointers; out may be NULL
 * to query the sizes.  out_len is the capacity of out. */
int chia_attn_tile_map(const chia_attn_args* args, int32_t residue,
                       int32_t rows_per_block, int32_t* n_qb, int32_t* n_kt,
                       int8_t* out, int64_t out_len);

/* Per-query visible key interval for one residue class (host-only, for tests):
 * writes jlo[i'], jhi[i'] (sub-sequence coordinates) and the prefix length.
 * len must be >= the residue's sub-sequence length. */
int chia_attn_query_intervals(const chia_attn_args* args, int32_t residue,
                              int32_t* jlo, int32_t* jhi, int32_t* prefix_len,
                              int64_t len);

const char* chia_attn_status_string(int status);
int chia_attn_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* CHIA_ATTN_H */
