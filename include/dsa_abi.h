/*
 * dsa_abi.h -- C ABI of the MI355X (gfx950) DeepSeek sparse attention (DSA)
 * library libdsa_amd.so.
 *
 * Every entry point takes plain device pointers, element strides and sizes;
 * no framework types cross this boundary.  Calls enqueue work on `stream`
 * (a hipStream_t; NULL = the default stream), never synchronize, never
 * allocate and never free.  Status 0 = success; otherwise dsa_last_error()
 * (thread-local) describes the failure.
 *
 * Reference interfaces replaced (Starkdoorstep12/flashinfer-repo):
 *   dsa_attn_fwd          solution/triton/kernel.py:138-182   kernel()
 *                         solution/triton/kernel.py:496-567   kernel_splitk()
 *                         solution/triton/kernel.py:707-799   kernel_splitk_v2()
 *                         (its split partial kernel.py:343-434 and merges
 *                         kernel.py:437-493, 583-704 run inside this call)
 *   dsa_indexer_topk      solution/triton/indexer_kernel.py:345-433
 *                         run_indexer_and_topk() (score kernel :4-287, top-k
 *                         kernel :289-343)
 *   dsa_attn_fwd_partial  solution/triton/kernel.py:343-434  dsa_fwd_kernel_splitk
 *   dsa_attn_merge        solution/triton/kernel.py:437-493  dsa_reduce_kernel
 *   dsa_attn_workspace_bytes / dsa_indexer_workspace_bytes
 *                         replace the per-call torch.zeros scratch of
 *                         kernel.py:526-528 and indexer_kernel.py:376-378
 *                         with a caller-owned workspace.
 *   dsa_indexer_k_append  no kernel in the reference: writes the paged fp8
 *                         indexer K cache that indexer_kernel.py:163-197
 *                         reads (quantise-on-append).
 *   dsa_indexer_prepare_k / dsa_indexer_k_planes_bytes /
 *   dsa_indexer_workspace_bytes_prepared
 *                         no counterpart: K operand planes kept beside the K
 *                         cache, so a call skips the per-call re-read of K
 *                         that indexer_kernel.py:185-275 does.
 *   dsa_attn_counter_bytes / dsa_attn_call_counter_bytes
 *                         no counterpart: size of the optional split
 *                         counters of dsa_attn_fwd (for any call of a head
 *                         count / for one call shape).
 */
#ifndef DSA_ABI_H
#define DSA_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DSA_ABI_VERSION 5

#define DSA_OK 0
#define DSA_EINVAL 1      /* bad pointer, size, stride or alignment */
#define DSA_EUNSUPPORTED 2 /* shape outside what the kernels implement */
#define DSA_ELAUNCH 3     /* HIP launch failure */
#define DSA_EWORKSPACE 4  /* workspace missing or too small */

/*
 * Sparse MLA attention over top-k selected cache slots
 * (kernel.py:138-143 tensor contract; golden semantics
 * indexer_kernel.py:436-497).
 *
 *   q_nope [T,H,head_dim_ckv] bf16, q_pe [T,H,head_dim_kpe] bf16
 *   ckv    [num_pages,page_size,head_dim_ckv] bf16
 *   kpe    [num_pages,page_size,head_dim_kpe] bf16
 *   sparse_indices [T,topk] int32: slot id = page*page_size + offset;
 *            -1 (and any id outside [0, num_pages*page_size)) is padding
 *   output [T,H,head_dim_ckv] bf16, lse [T,H] fp32 (base 2; -inf and a zero
 *            output row for a token with no valid slot)
 *
 * Strides are in elements; the last dimension of every tensor is contiguous
 * and rows must be 16-byte aligned.  head_dim_ckv must be 512, head_dim_kpe
 * 64 and H a multiple of 16.  num_splits: 0 = automatic (fills the GPU),
 * otherwise the number of top-k chunks computed in parallel per token and
 * merged with log-sum-exp weights in a fixed order (results are
 * deterministic).  A chunk holds at most 2048 entries, so longer rows always
 * run split (the count is raised to ceil(topk / 2048));
 * dsa_attn_num_splits() gives the count.  A split
 * call needs dsa_attn_workspace_bytes() of workspace (16-byte aligned, contents
 * irrelevant) for the fp32 partials.
 *
 * split_counters (optional, no counterpart in the reference): with NULL a
 * split call runs a second kernel that merges the partials (the reference's
 * kernel_splitk launch pair, kernel.py:534 and :555).  Where
 * dsa_attn_counter_bytes() is not 0 (head counts of an odd number of 16-head
 * groups, e.g. H=16 decode), the call has at most 4 splits (more are merged
 * faster by the second kernel) and that much 4-byte aligned, all-zero memory
 * is given, the merge happens inside the attention kernel instead (the
 * workgroup that finishes a token's chunk last merges it; same bits as the
 * two-kernel path) and every call that completes leaves the counters zero
 * again, so zero them once (e.g. hipMemset) and reuse them for calls of any
 * shape.  Otherwise the counters are ignored.  Calls that run concurrently
 * must share neither a workspace nor counters.
 */
typedef struct dsa_attn_args {
  const void *q_nope;
  int64_t q_nope_stride_t, q_nope_stride_h;
  const void *q_pe;
  int64_t q_pe_stride_t, q_pe_stride_h;
  const void *ckv;
  int64_t ckv_stride_page, ckv_stride_tok;
  const void *kpe;
  int64_t kpe_stride_page, kpe_stride_tok;
  const int32_t *sparse_indices;
  int64_t idx_stride_t;
  void *output;
  int64_t out_stride_t, out_stride_h;
  float *lse;
  int64_t lse_stride_t, lse_stride_h;
  int64_t num_tokens, num_heads, topk;
  int64_t page_size, num_pages;
  int64_t head_dim_ckv, head_dim_kpe;
  float sm_scale;
  int32_t num_splits;
  void *workspace;
  size_t workspace_bytes;
  uint32_t *split_counters;
  size_t split_counters_bytes;
} dsa_attn_args;

int dsa_attn_fwd(const dsa_attn_args *args, void *stream);

/*
 * dsa_attn_fwd without a caller workspace: no counterpart in the reference.
 * For callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments and results as dsa_attn_fwd, except that workspace and
 * split_counters must be NULL: a split call keeps its fp32 partials in a
 * device array of DSA_NOALLOC_SCRATCH_BYTES that the library owns (one per
 * device, held until the process ends) and merges them with the separate
 * merge kernel.  With num_splits = 0 the call takes the automatic split count
 * or, when that count's workspace (dsa_attn_workspace_bytes) is larger than
 * the array, the most splits below it whose workspace fits (one split needs
 * none); an explicit num_splits whose workspace is larger fails with
 * DSA_EWORKSPACE.  The call allocates and frees nothing.  Its first call on
 * a device looks up the array's address (with the calling thread's stream
 * capture mode relaxed for that lookup, so it may run under graph capture).
 * Calls that overlap on one device share the array and race.
 */
#define DSA_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)

int dsa_attn_fwd_noalloc(const dsa_attn_args *args, void *stream);

/* Split count dsa_attn_fwd will use for this shape (requested 0 = auto). */
int32_t dsa_attn_num_splits(int64_t num_tokens, int64_t num_heads, int64_t topk,
                            int32_t requested);

/* Workspace dsa_attn_fwd needs (0 when one split suffices). */
size_t dsa_attn_workspace_bytes(int64_t num_tokens, int64_t num_heads, int64_t topk,
                                int32_t requested_splits);

/* Size of dsa_attn_args.split_counters for num_tokens tokens of num_heads
 * heads (any top-k and split count); 0 when calls with this head count always
 * merge with the separate kernel. */
size_t dsa_attn_counter_bytes(int64_t num_tokens, int64_t num_heads);

/* Split counters one call of this shape actually uses (requested_splits as in
 * dsa_attn_args.num_splits): dsa_attn_counter_bytes(num_tokens, num_heads)
 * when the call merges its splits inside the attention kernel (2 to 4
 * splits, an odd number of 16-head groups), else 0 -- the call then runs the
 * separate merge kernel and never touches counters.  No counterpart in the
 * reference. */
size_t dsa_attn_call_counter_bytes(int64_t num_tokens, int64_t num_heads, int64_t topk,
                                   int32_t requested_splits);

/*
 * The two halves of a split dsa_attn_fwd, for callers that merge partials
 * themselves -- e.g. a cache sharded by slot ranges over several devices
 * (each shard computes partials over its own slots, the partials are
 * gathered, one dsa_attn_merge finishes) -- or that time the halves apart.
 * Reference: the split partial kernel.py:343-434 and its merge
 * kernel.py:437-493 (the separate launches of kernel_splitk, :534 and :555).
 *
 * dsa_attn_fwd_partial takes the same arguments as dsa_attn_fwd (output and
 * lse are not touched and may be NULL) and writes, for every split count
 * including 1, into the workspace (dsa_attn_partial_bytes() bytes):
 *   part_acc = (float*)workspace              [T, S, H, 512]
 *   part_ml  = part_acc + T*S*H*512           [T, S, H, 2]
 * where for chunk s of token t and head h, with x_j the scaled logits of the
 * chunk's valid slots: m = part_ml[...][0] is a reference value (in log2
 * units) with every 2^(x_j*log2(e) - m) <= 256, l = part_ml[...][1] =
 * sum_j 2^(x_j*log2(e) - m) and part_acc = sum_j 2^(x_j*log2(e) - m) *
 * ckv[s_j].  A chunk without valid slots has m = -inf, l = 0, acc = 0.
 *
 * dsa_attn_merge combines num_splits such partials per (token, head) in
 * split order: out = sum_s 2^(m_s - M) acc_s / sum_s 2^(m_s - M) l_s,
 * lse = M + log2(sum_s 2^(m_s - M) l_s), M = max_s m_s (zeros / -inf when
 * every chunk is empty).
 */
int dsa_attn_fwd_partial(const dsa_attn_args *args, void *stream);

size_t dsa_attn_partial_bytes(int64_t num_tokens, int64_t num_heads, int64_t topk,
                              int32_t requested_splits);

typedef struct dsa_attn_merge_args {
  const float *part_acc; /* [T, S, H, 512] fp32, 16-byte aligned */
  const float *part_ml;  /* [T, S, H, 2] fp32 */
  int64_t num_tokens, num_splits, num_heads;
  void *output; /* [T, H, 512] bf16, element strides below */
  int64_t out_stride_t, out_stride_h;
  float *lse; /* [T, H] */
  int64_t lse_stride_t, lse_stride_h;
} dsa_attn_merge_args;

int dsa_attn_merge(const dsa_attn_merge_args *args, void *stream);

/*
 * Lightning indexer + top-k (indexer_kernel.py:345-433 interface; score
 * structure :185-275; selection as :289-343 intends):
 *
 *   score[t,s] = sum_h w[t,h] * relu(q[t,h,:] . k[s,:] * k_scale[s])
 *
 * computed in the factored form k_scale[s] * sum_h w[t,h] * relu(dot), which
 * is equal for the positive scales quantisation produces, with one exact
 * rounding order: D_h = 2^18 * (exact dot of the e4m3fn values; NaN codes count
 * as 0); r_h = fl32(max(D_h, 0)); the heads form 4 groups of num_heads/4
 * consecutive heads and group g sums G_g = fma(w[t,h], r_h, G_g) in ascending
 * head order from 0; total = fl32(fl32(G_0 + G_1) + fl32(G_2 + G_3));
 * score = fl32(total * fl32(k_scale[s] * 2^-18)).
 * Position s is a candidate for row t iff s <= causal_limit[t].  The k
 * largest candidates are selected, ties to the lower position; rows with
 * fewer candidates are padded with -1.  Output order is ascending position.
 * If block_table is non-NULL the output holds physical slots
 * block_table[t*block_table_stride + s/page_size]*page_size + s%page_size.
 *
 *   q_idx [T,num_heads,head_dim] e4m3fn codes, k_idx [S,head_dim] e4m3fn
 *   codes (both 16-byte aligned), k_scale [S] fp32, weights [T,num_heads]
 *   fp32, causal_limit [T] int32, out [T,topk] int32; scores_out [T,S] fp32
 *   optional (NULL = not returned; masked entries hold -inf).
 * head_dim must be 128, num_heads 16, 32, 48 or 64, topk <= 2^24.  The
 * workspace (dsa_indexer_workspace_bytes, 256-byte aligned) holds the MFMA
 * operand pieces of k and, unless scores_out is given, the scores (the q
 * operands are derived inside the score kernel); a call whose workspace
 * size is 0 may pass NULL.
 */
typedef struct dsa_indexer_args {
  const uint8_t *q_idx;
  const uint8_t *k_idx;
  const float *k_scale;
  const float *weights;
  const int32_t *causal_limit;
  int64_t num_tokens, num_heads, head_dim, num_positions, topk;
  const int32_t *block_table;
  int64_t block_table_stride, page_size;
  int32_t *out;
  float *scores_out;
  void *workspace;
  size_t workspace_bytes;
  /* Optional paged fp8 K cache (then k_idx and k_scale are NULL): position
   * s is token s % k_page_size of page k_pages[s / k_page_size] of k_cache
   * (layout below); k_page_size a multiple of 4, k_cache 16-byte aligned. */
  const uint8_t *k_cache;
  const int32_t *k_pages;
  int64_t k_page_size;
  /* Entries per block-table row (required with block_table: at least
   * ceil(num_positions / page_size), the pages a selected position can
   * fall in). */
  int64_t block_table_width;
  /* Pages of k_cache (required with k_cache, >= 1).  A position whose
   * k_pages entry lies outside [0, k_num_pages) reads as a zero row with a
   * zero scale (its score is 0); nothing outside k_cache is read. */
  int64_t k_num_pages;
  /* Optional prepared K planes (ABI version 5; no counterpart in the
   * reference): a buffer that dsa_indexer_prepare_k filled for at least these
   * num_positions positions, laid out for k_planes_capacity >= num_positions
   * positions (256-byte aligned, dsa_indexer_k_planes_bytes(capacity) bytes).
   * The call then reads the K operands from it and does no K preparation;
   * k_idx, k_scale and k_cache are ignored and may be NULL, and the workspace
   * needs only dsa_indexer_workspace_bytes_prepared() bytes. */
  const void *k_planes;
  int64_t k_planes_capacity;
} dsa_indexer_args;

int dsa_indexer_topk(const dsa_indexer_args *args, void *stream);

/*
 * Prepared K planes (no counterpart in the reference, whose score kernel
 * re-reads and dequantises K on every call, indexer_kernel.py:185-275).  The
 * K cache changes only where tokens are appended, so the MFMA operand planes
 * the score kernel reads (per 16-position block: the e4m3 values as signed
 * 7-bit pieces in MFMA lane order, the block's largest magnitude, and
 * fl32(k_scale * 2^-18) per position) can be derived once and kept beside
 * the cache.  dsa_indexer_prepare_k (re)derives the blocks that hold
 * positions [first_position, first_position + count) of a sequence of
 * num_positions positions (flat k_idx/k_scale, or a paged K cache read
 * through k_pages as in dsa_indexer_args; a block's positions at or past
 * num_positions read as zeros), into a planes buffer laid out for
 * k_planes_capacity positions.  After an append, re-preparing the appended
 * positions keeps the planes current; calls of dsa_indexer_topk with those
 * planes give the same bits as calls that prepare K themselves.
 */
typedef struct dsa_indexer_k_prepare_args {
  const uint8_t *k_idx;     /* [num_positions, 128] e4m3fn codes, or NULL (paged) */
  const float *k_scale;     /* [num_positions] */
  const uint8_t *k_cache;   /* paged cache (then k_idx, k_scale NULL) */
  const int32_t *k_pages;
  int64_t k_page_size, k_num_pages;
  int64_t num_positions;
  int64_t first_position, count;
  void *k_planes;           /* 256-byte aligned */
  int64_t k_planes_capacity;
} dsa_indexer_k_prepare_args;

size_t dsa_indexer_k_planes_bytes(int64_t capacity);

int dsa_indexer_prepare_k(const dsa_indexer_k_prepare_args *args, void *stream);

/*
 * Paged fp8 indexer K cache and its quantise-on-append (the K-cache format on
 * either side of the indexer; the reference's kernel reads a 129-element
 * record whose scale is one int8 element, indexer_kernel.py:163-197).  Page
 * p is k_page_size tokens of DSA_INDEXER_K_TOKEN_BYTES bytes: bytes
 * [0, 128*page_size) hold the e4m3fn codes of token o at o*128, bytes
 * [128*page_size, 132*page_size) its fp32 scale at 128*page_size + 4*o (the
 * codes of a page stay contiguous).  A slot id is page*page_size + offset.
 *
 * dsa_indexer_k_append quantises each bf16 row k[i, 0:128] to that format and
 * writes it to slot slots[i] (negative or out-of-range slots are skipped):
 *   amax = max_j |k[i,j]| (fp32), scale = fl32(max(amax, 1e-4f) / 448),
 *   code_j = e4m3fn, rounded to nearest even, of clamp(fl32(k[i,j] / scale),
 *   -448, 448).
 * Rows are 16-byte aligned with row stride k_stride elements; page_size a
 * multiple of 4 and k_cache 16-byte aligned.  Calls with overlapping slots
 * race like any concurrent writes.
 */
#define DSA_INDEXER_K_TOKEN_BYTES 132

typedef struct dsa_k_append_args {
  const void *k;          /* [num_tokens, 128] bf16 */
  int64_t k_stride;
  const int32_t *slots;   /* [num_tokens] */
  int64_t num_tokens;
  uint8_t *k_cache;       /* [num_pages, page_size * 132] */
  int64_t num_pages, page_size;
} dsa_k_append_args;

int dsa_indexer_k_append(const dsa_k_append_args *args, void *stream);

size_t dsa_indexer_workspace_bytes(int64_t num_tokens, int64_t num_heads, int64_t head_dim,
                                   int64_t num_positions);

/* Workspace of a dsa_indexer_topk call that reads prepared K planes: the
 * scores, unless scores_out is given. */
size_t dsa_indexer_workspace_bytes_prepared(int64_t num_tokens, int64_t num_heads,
                                            int64_t head_dim, int64_t num_positions);

/* Thread-local description of the last failure ("" if none). */
const char *dsa_last_error(void);

int dsa_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* DSA_ABI_H */
