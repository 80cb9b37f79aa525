// dsa_abi.cpp -- the extern "C" boundary of libdsa_amd.so (declared in
// include/dsa_abi.h).  Validates shapes, strides and alignment on the host,
// chooses the launch configuration from shapes alone (no device reads, no
// synchronisation, no allocation) and enqueues the HIP kernels on the
// caller's stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/dsa_abi.h"
#include "dsa_internal.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return DSA_OK;
}

bool aligned(const void *p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

constexpr int64_t kMaxWaveSplits = 16;

// Top-k chunk length per split and the split count that results.  Automatic
// mode aims for about one workgroup per compute unit while keeping enough
// work per chunk: four 32-key tiles for the shared-ring layouts.  The
// four-wave layout (every odd number of 16-head groups; an even number while
// T x groups <= 128, or <= 64 for multiples of 8 groups) takes the most splits that keep its T x S x groups
// workgroups within one round, at most kMaxWaveSplits and chunks of at least
// 64 keys (one 16-key block per wave).  Past that the shared-ring layouts,
// with the split count that fills one round of their workgroups.  Measured
// over H = 16..128, T = 1..64, every layout and split count (top-k 2048, and
// 256 for config 1): the fastest configuration of each shape was within
// about 1 us of a grid of about one workgroup per CU (H=16: T=1 16.3 -> 11.9
// us with 16 splits instead of 8; H=48 T=64 82.5 -> 54.6 us with 1 split
// instead of 4).  An explicit
// request is honoured up to one key per split (the reference's kernel_splitk
// additionally required topk % SPLIT_K == 0, kernel.py:512; uneven chunks are
// fine here).  Either way a chunk never exceeds the layout's maximum, so very
// long rows get extra splits.
void choose_splits(int64_t T, int64_t H, int64_t K, int32_t requested, int32_t *splits,
                   int32_t *chunk) {
  if (K <= 0) {
    *splits = 1;
    *chunk = 0;
    return;
  }
  int64_t S;
  int64_t c;
  const int64_t min_s = ceil_div(K, dsa::attn_max_chunk((int)H));
  if (requested > 0) {
    S = requested < K ? requested : K;
    if (S < min_s) S = min_s;
    c = ceil_div(K, S);
  } else {
    const int64_t groups = H / dsa::kHeadsPerGroup > 0 ? H / dsa::kHeadsPerGroup : 1;
    const int64_t Tn = T > 0 ? T : 1;
    const int64_t tiles = ceil_div(K, dsa::kKeysPerTile);
    int64_t max_s;
    // the four-wave layout while it gets at least 2 splits (at least 4 for
    // multiples of 8 groups, whose four-wave ring layout is faster at 2:
    // H=128 T=16 35.1 us with 8 splits against 36.8 us)
    if (groups % 2 != 0 || Tn * groups <= dsa::kNumCU / (groups % 8 == 0 ? 4 : 2)) {
      // four-wave layout, T x S x groups workgroups within one round
      S = dsa::kNumCU / (Tn * groups);
      max_s = std::min<int64_t>(ceil_div(K, 64), kMaxWaveSplits);
    } else if (groups % 8 == 0 && Tn * (groups / 4) <= dsa::kNumCU / 2) {
      // workgroups of four head groups, within one round
      S = dsa::kNumCU / (Tn * (groups / 4));
      max_s = ceil_div(tiles, dsa::kMinTilesPerSplit);
    } else {
      // workgroups of 8 (groups % 8 == 0), 4 or 2 head groups
      const int64_t per = groups % 8 == 0 ? 8 : groups % 4 == 0 ? 4 : 2;
      S = ceil_div(dsa::kNumCU, Tn * (groups / per));
      max_s = ceil_div(tiles, dsa::kMinTilesPerSplit);
    }
    if (S > max_s) S = max_s;
    if (S < min_s) S = min_s;
    if (S < 1) S = 1;
    c = ceil_div(tiles, S) * dsa::kKeysPerTile;
  }
  S = ceil_div(K, c);
  *splits = (int32_t)S;
  *chunk = (int32_t)c;
}

// Partials of dsa_attn_fwd_partial: [partial outputs T x S x H x 512 fp32]
// [(max, sum) T x S x H fp32].
size_t partial_bytes(int64_t T, int64_t H, int32_t S) {
  const size_t rows = (size_t)T * (size_t)S * (size_t)H;
  return rows * dsa::kHeadDimCkv * sizeof(float) + rows * 2 * sizeof(float);
}

// Workspace of a split dsa_attn_fwd: the same partial outputs, then room for
// the in-kernel merge's (max, sum) copies, one per feature slice (T x S x H x 8).
size_t attn_workspace(int64_t T, int64_t H, int32_t S) {
  const size_t rows = (size_t)T * (size_t)S * (size_t)H;
  return S <= 1 ? 0 : rows * dsa::kHeadDimCkv * sizeof(float) + rows * 16 * sizeof(float);
}

}  // namespace

extern "C" {

const char *dsa_last_error(void) { return g_last_error.c_str(); }

int dsa_abi_version(void) { return DSA_ABI_VERSION; }

int32_t dsa_attn_num_splits(int64_t num_tokens, int64_t num_heads, int64_t topk,
                            int32_t requested) {
  int32_t s, c;
  choose_splits(num_tokens, num_heads, topk, requested, &s, &c);
  return s;
}

size_t dsa_attn_workspace_bytes(int64_t num_tokens, int64_t num_heads, int64_t topk,
                                int32_t requested_splits) {
  int32_t s, c;
  choose_splits(num_tokens, num_heads, topk, requested_splits, &s, &c);
  return attn_workspace(num_tokens, num_heads, s);
}

size_t dsa_attn_counter_bytes(int64_t num_tokens, int64_t num_heads) {
  if (num_tokens <= 0 || num_heads < dsa::kHeadsPerGroup || num_heads > 4096 ||
      !dsa::attn_merges_in_kernel((int)num_heads, 2))
    return 0;
  return (size_t)dsa::attn_counter_words(num_tokens, dsa::attn_head_blocks((int)num_heads)) *
         sizeof(uint32_t);
}

size_t dsa_attn_call_counter_bytes(int64_t num_tokens, int64_t num_heads, int64_t topk,
                                   int32_t requested_splits) {
  if (requested_splits < 0 || num_heads < dsa::kHeadsPerGroup || num_heads > 4096) return 0;
  int32_t s, c;
  choose_splits(num_tokens, num_heads, topk, requested_splits, &s, &c);
  if (s < 2 || !dsa::attn_merges_in_kernel((int)num_heads, s)) return 0;
  return dsa_attn_counter_bytes(num_tokens, num_heads);
}

}  // extern "C"

namespace {

// Validates an attention call and fills the kernel parameters.  With
// partial_only the fp32 partials are written (and required) for every split
// count, and the workspace must hold them.
int prepare_attn(const char *fn, const dsa_attn_args *a, bool partial_only, dsa::AttnParams *p) {
  if (!a) return fail(DSA_EINVAL, "%s: args is NULL", fn);
  if (a->head_dim_ckv != dsa::kHeadDimCkv || a->head_dim_kpe != dsa::kHeadDimKpe)
    return fail(DSA_EUNSUPPORTED, "%s: head dims must be ckv=512, kpe=64 (got %lld, %lld)", fn,
                (long long)a->head_dim_ckv, (long long)a->head_dim_kpe);
  if (a->num_tokens < 0 || a->num_heads <= 0 || a->topk < 0 || a->page_size <= 0 ||
      a->num_pages < 0)
    return fail(DSA_EINVAL, "%s: negative or zero size (T=%lld H=%lld topk=%lld "
                "page_size=%lld num_pages=%lld)", fn, (long long)a->num_tokens,
                (long long)a->num_heads, (long long)a->topk, (long long)a->page_size,
                (long long)a->num_pages);
  if (a->num_heads % dsa::kHeadsPerGroup != 0)
    return fail(DSA_EUNSUPPORTED, "%s: num_heads must be a multiple of 16 (got %lld)", fn,
                (long long)a->num_heads);
  if (a->num_tokens > (1 << 26) || a->topk > (1 << 30) || a->num_heads > 4096 ||
      a->page_size > (1 << 30))
    return fail(DSA_EUNSUPPORTED, "%s: size beyond the supported range", fn);
  if (a->num_splits < 0) return fail(DSA_EINVAL, "%s: num_splits must be >= 0", fn);
  if (a->num_tokens == 0) return DSA_OK;
  if (!a->q_nope || !a->q_pe || (!partial_only && (!a->output || !a->lse)) ||
      (a->topk > 0 && !a->sparse_indices))
    return fail(DSA_EINVAL, "%s: NULL tensor pointer", fn);
  if (a->num_pages > 0 && (!a->ckv || !a->kpe))
    return fail(DSA_EINVAL, "%s: NULL cache pointer", fn);
  // 16-byte rows for the MFMA operand loads and the LDS DMA gathers.
  if (!aligned(a->q_nope, 16) || !aligned(a->q_pe, 16) || !aligned(a->ckv, 16) ||
      !aligned(a->kpe, 16) || (a->q_nope_stride_t * 2) % 16 || (a->q_nope_stride_h * 2) % 16 ||
      (a->q_pe_stride_t * 2) % 16 || (a->q_pe_stride_h * 2) % 16 ||
      (a->ckv_stride_page * 2) % 16 || (a->ckv_stride_tok * 2) % 16 ||
      (a->kpe_stride_page * 2) % 16 || (a->kpe_stride_tok * 2) % 16)
    return fail(DSA_EINVAL, "%s: q/ckv/kpe rows must be 16-byte aligned", fn);
  if (!partial_only && (!aligned(a->output, 8) || (a->out_stride_t * 2) % 8 ||
                        (a->out_stride_h * 2) % 8 || !aligned(a->lse, 4)))
    return fail(DSA_EINVAL, "%s: output rows must be 8-byte aligned", fn);
  if (!aligned(a->sparse_indices, 4))
    return fail(DSA_EINVAL, "%s: sparse_indices must be 4-byte aligned", fn);

  int32_t S, chunk;
  choose_splits(a->num_tokens, a->num_heads, a->topk, a->num_splits, &S, &chunk);
  if (a->num_tokens * (int64_t)S > 0x7fffffffLL)
    return fail(DSA_EUNSUPPORTED, "%s: num_tokens * splits exceeds the grid", fn);
  const size_t need = partial_only ? partial_bytes(a->num_tokens, a->num_heads, S)
                                   : attn_workspace(a->num_tokens, a->num_heads, S);
  if (need > 0 && (!a->workspace || a->workspace_bytes < need || !aligned(a->workspace, 16)))
    return fail(DSA_EWORKSPACE, "%s: workspace of %zu bytes (16-byte aligned) needed, got %zu",
                fn, need, a->workspace ? a->workspace_bytes : (size_t)0);
  const bool merge_in_kernel = !partial_only && S > 1 && a->split_counters != nullptr &&
                               dsa::attn_merges_in_kernel((int)a->num_heads, S);
  if (merge_in_kernel) {
    const size_t cneed = (size_t)dsa::attn_counter_words(
                             a->num_tokens, dsa::attn_head_blocks((int)a->num_heads)) *
                         sizeof(uint32_t);
    if (a->split_counters_bytes < cneed || !aligned(a->split_counters, 4))
      return fail(DSA_EWORKSPACE, "%s: split_counters of %zu bytes (4-byte aligned) needed, got %zu",
                  fn, cneed, a->split_counters_bytes);
  }

  p->q_nope = static_cast<const char *>(a->q_nope);
  p->qn_st = a->q_nope_stride_t * 2;
  p->qn_sh = a->q_nope_stride_h * 2;
  p->q_pe = static_cast<const char *>(a->q_pe);
  p->qp_st = a->q_pe_stride_t * 2;
  p->qp_sh = a->q_pe_stride_h * 2;
  p->ckv = static_cast<const char *>(a->ckv);
  p->ckv_sp = a->ckv_stride_page * 2;
  p->ckv_so = a->ckv_stride_tok * 2;
  p->kpe = static_cast<const char *>(a->kpe);
  p->kpe_sp = a->kpe_stride_page * 2;
  p->kpe_so = a->kpe_stride_tok * 2;
  p->idx = a->sparse_indices;
  p->idx_st = a->idx_stride_t;
  p->out = static_cast<char *>(a->output);
  p->out_st = a->out_stride_t * 2;
  p->out_sh = a->out_stride_h * 2;
  p->lse = a->lse;
  p->lse_st = a->lse_stride_t;
  p->lse_sh = a->lse_stride_h;
  p->T = (int32_t)a->num_tokens;
  p->H = (int32_t)a->num_heads;
  p->K = (int32_t)a->topk;
  p->page_size = (int32_t)a->page_size;
  p->num_slots = a->num_pages * a->page_size;
  {
    int sh = 0;
    while ((int64_t(1) << sh) < a->page_size) ++sh;
    p->ps_shift = sh;
    p->ps_magic = (uint32_t)(((uint64_t)1 << (31 + sh)) / (uint64_t)a->page_size + 1);
  }
  {
    // Narrow addressing: dense caches (a page is page_size consecutive rows,
    // or pages of one row) whose extents stay below 2^31 bytes.
    const int64_t ps = a->page_size;
    const int64_t crs = ps == 1 ? p->ckv_sp : p->ckv_so, krs = ps == 1 ? p->kpe_sp : p->kpe_so;
    const bool dense = ps == 1 || (p->ckv_sp == ps * p->ckv_so && p->kpe_sp == ps * p->kpe_so);
    const int64_t n = p->num_slots;
    p->narrow = dense && crs > 0 && krs > 0 && crs < (1 << 24) && krs < (1 << 24) &&
                n < (1 << 24) && n * crs <= 0x7fffffffLL && n * krs <= 0x7fffffffLL;
    p->ckv_rs = p->narrow ? (uint32_t)crs : 0;
    p->kpe_rs = p->narrow ? (uint32_t)krs : 0;
    p->ckv_extent = p->narrow ? (uint32_t)(n * crs) : 0;
    p->kpe_extent = p->narrow ? (uint32_t)(n * krs) : 0;
  }
  p->scale_log2 = a->sm_scale * 1.4426950408889634f;
  p->num_splits = S;
  p->chunk = chunk;
  float *ws = static_cast<float *>(a->workspace);
  p->part_acc = ws;
  p->part_ml = ws ? ws + (size_t)a->num_tokens * S * a->num_heads * dsa::kHeadDimCkv : nullptr;
  p->partial_only = partial_only ? 1 : 0;
  p->counters = merge_in_kernel ? a->split_counters : nullptr;
  return DSA_OK;
}

}  // namespace

namespace dsa {

int attn_fwd(const char *fn, const dsa_attn_args *a, void *stream) {
  AttnParams p = {};
  const int rc = prepare_attn(fn, a, false, &p);
  if (rc != DSA_OK) return rc;
  if (a->num_tokens == 0) return ok();
  const hipError_t e = launch_attention(p, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(DSA_ELAUNCH, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return ok();
}

int set_error(int code, const char *msg) { return fail(code, "%s", msg); }

size_t attn_split_workspace(int64_t T, int64_t H, int64_t K, int32_t requested) {
  int32_t s, c;
  choose_splits(T, H, K, requested, &s, &c);
  return attn_workspace(T, H, s);
}

}  // namespace dsa

extern "C" {

int dsa_attn_fwd(const dsa_attn_args *a, void *stream) {
  return dsa::attn_fwd("dsa_attn_fwd", a, stream);
}

int dsa_attn_fwd_partial(const dsa_attn_args *a, void *stream) {
  dsa::AttnParams p = {};
  const int rc = prepare_attn("dsa_attn_fwd_partial", a, true, &p);
  if (rc != DSA_OK) return rc;
  if (a->num_tokens == 0) return ok();
  const hipError_t e = dsa::launch_attention_partial(p, static_cast<hipStream_t>(stream));
  if (e != hipSuccess)
    return fail(DSA_ELAUNCH, "dsa_attn_fwd_partial: launch failed: %s", hipGetErrorString(e));
  return ok();
}

size_t dsa_attn_partial_bytes(int64_t num_tokens, int64_t num_heads, int64_t topk,
                              int32_t requested_splits) {
  int32_t s, c;
  choose_splits(num_tokens, num_heads, topk, requested_splits, &s, &c);
  return partial_bytes(num_tokens, num_heads, s);
}

int dsa_attn_merge(const dsa_attn_merge_args *a, void *stream) {
  if (!a) return fail(DSA_EINVAL, "dsa_attn_merge: args is NULL");
  if (a->num_tokens < 0 || a->num_splits <= 0 || a->num_heads <= 0 ||
      a->num_tokens * a->num_splits > 0x7fffffffLL || a->num_heads > 65535)
    return fail(DSA_EINVAL, "dsa_attn_merge: bad sizes (T=%lld S=%lld H=%lld)",
                (long long)a->num_tokens, (long long)a->num_splits, (long long)a->num_heads);
  if (a->num_tokens == 0) return ok();
  if (!a->part_acc || !a->part_ml || !a->output || !a->lse)
    return fail(DSA_EINVAL, "dsa_attn_merge: NULL pointer");
  if (!aligned(a->part_acc, 16) || !aligned(a->part_ml, 8) || !aligned(a->output, 8) ||
      (a->out_stride_t * 2) % 8 || (a->out_stride_h * 2) % 8 || !aligned(a->lse, 4))
    return fail(DSA_EINVAL, "dsa_attn_merge: misaligned pointer or stride");
  dsa::AttnParams p = {};
  p.T = (int32_t)a->num_tokens;
  p.H = (int32_t)a->num_heads;
  p.num_splits = (int32_t)a->num_splits;
  p.part_acc = const_cast<float *>(a->part_acc);
  p.part_ml = const_cast<float *>(a->part_ml);
  p.out = static_cast<char *>(a->output);
  p.out_st = a->out_stride_t * 2;
  p.out_sh = a->out_stride_h * 2;
  p.lse = a->lse;
  p.lse_st = a->lse_stride_t;
  p.lse_sh = a->lse_stride_h;
  const hipError_t e = dsa::launch_attention_merge(p, static_cast<hipStream_t>(stream));
  if (e != hipSuccess)
    return fail(DSA_ELAUNCH, "dsa_attn_merge: launch failed: %s", hipGetErrorString(e));
  return ok();
}

}  // extern "C"

// ---- indexer -------------------------------------------------------------

namespace {
constexpr int64_t kIndexerHeadDim = 128;
constexpr int64_t kIndexerMaxHeads = 64;

size_t up256(size_t x) { return (x + 255) / 256 * 256; }
}  // namespace

namespace dsa {
IndexerWorkspace indexer_workspace_layout(int64_t T, int64_t Hi, int64_t S, bool own_scores,
                                          bool own_k) {
  IndexerWorkspace w = {};
  (void)Hi;
  const size_t kblocks = own_k ? (size_t)(S + 15) / 16 : 0;
  size_t off = 0;
  w.k_pieces = off;
  off += up256(kblocks * 3 * 2 * 1024);
  w.k_max = off;
  off += up256(kblocks * 4);
  w.k_cs = off;
  if (own_k) off += up256((size_t)S * 4);
  w.scores = off;
  if (own_scores) off += up256((size_t)T * (size_t)S * 4);
  w.total = off;
  return w;
}

KPlanesLayout k_planes_layout(int64_t C) {
  KPlanesLayout l = {};
  const size_t kblocks = (size_t)(C + 15) / 16;
  l.k_pieces = 0;
  l.k_max = up256(kblocks * 3 * 2 * 1024);
  l.k_cs = l.k_max + up256(kblocks * 4);
  l.total = l.k_cs + up256((size_t)C * 4);
  return l;
}
}  // namespace dsa

extern "C" {

size_t dsa_indexer_workspace_bytes(int64_t num_tokens, int64_t num_heads, int64_t head_dim,
                                   int64_t num_positions) {
  if (num_tokens < 0 || num_heads < 0 || head_dim < 0 || num_positions < 0) return 0;
  return dsa::indexer_workspace_layout(num_tokens, num_heads, num_positions, true, true).total;
}

size_t dsa_indexer_workspace_bytes_prepared(int64_t num_tokens, int64_t num_heads,
                                            int64_t head_dim, int64_t num_positions) {
  if (num_tokens < 0 || num_heads < 0 || head_dim < 0 || num_positions < 0) return 0;
  return dsa::indexer_workspace_layout(num_tokens, num_heads, num_positions, true, false).total;
}

size_t dsa_indexer_k_planes_bytes(int64_t capacity) {
  if (capacity < 0 || capacity > 0x7fffffffLL) return 0;
  return dsa::k_planes_layout(capacity).total;
}

int dsa_indexer_topk(const dsa_indexer_args *a, void *stream) {
  const char *fn = "dsa_indexer_topk";
  if (!a) return fail(DSA_EINVAL, "%s: args is NULL", fn);
  if (a->head_dim != kIndexerHeadDim)
    return fail(DSA_EUNSUPPORTED, "%s: head_dim must be 128 (got %lld)", fn, (long long)a->head_dim);
  if (a->num_heads <= 0 || a->num_heads % 16 != 0 || a->num_heads > kIndexerMaxHeads)
    return fail(DSA_EUNSUPPORTED, "%s: num_heads must be 16, 32, 48 or 64 (got %lld)", fn,
                (long long)a->num_heads);
  if (a->num_tokens < 0 || a->num_positions < 0 || a->topk < 0)
    return fail(DSA_EINVAL, "%s: negative size", fn);
  if (a->num_tokens > (1 << 24) || a->num_positions > 0x7fffffffLL || a->topk > (1 << 24) ||
      a->num_tokens * a->num_positions > (1LL << 40))
    return fail(DSA_EUNSUPPORTED, "%s: size beyond the supported range", fn);
  if (a->num_tokens == 0) return ok();
  const bool prepared = a->k_planes != nullptr;
  const bool paged = !prepared && a->k_cache != nullptr;
  if (paged && (a->k_idx || a->k_scale))
    return fail(DSA_EINVAL, "%s: give k_idx/k_scale or k_cache, not both", fn);
  if (paged && (!a->k_pages || a->k_page_size <= 0 || a->k_page_size % 4 != 0 ||
                a->k_page_size > (1 << 24)))
    return fail(DSA_EINVAL, "%s: k_cache needs k_pages and a k_page_size that is a positive "
                "multiple of 4 (got %lld)", fn, (long long)a->k_page_size);
  if (!a->q_idx || !a->weights || !a->causal_limit || (a->topk > 0 && !a->out) ||
      (a->num_positions > 0 && !paged && !prepared && (!a->k_idx || !a->k_scale)))
    return fail(DSA_EINVAL, "%s: NULL tensor pointer", fn);
  if (!aligned(a->q_idx, 16) || !aligned(a->k_idx, 16) || !aligned(a->k_scale, 4) ||
      !aligned(a->weights, 4) || !aligned(a->causal_limit, 4) || !aligned(a->out, 4) ||
      !aligned(a->scores_out, 4) || !aligned(a->k_cache, 16) || !aligned(a->k_pages, 4))
    return fail(DSA_EINVAL, "%s: misaligned pointer (e4m3 rows need 16 bytes)", fn);
  if (a->block_table && (a->page_size <= 0 || a->block_table_stride < 0))
    return fail(DSA_EINVAL, "%s: block_table needs page_size > 0 and a stride >= 0", fn);
  if (a->block_table && a->block_table_width < ceil_div(a->num_positions, a->page_size))
    return fail(DSA_EINVAL, "%s: block_table rows hold %lld pages, %lld positions of page size "
                "%lld need %lld", fn, (long long)a->block_table_width,
                (long long)a->num_positions, (long long)a->page_size,
                (long long)ceil_div(a->num_positions, a->page_size));
  if (a->block_table && a->block_table_stride > 0 &&
      a->block_table_stride < a->block_table_width)
    return fail(DSA_EINVAL, "%s: block_table stride %lld is below its width %lld", fn,
                (long long)a->block_table_stride, (long long)a->block_table_width);
  if (paged && (a->k_num_pages <= 0 || a->k_num_pages > 0x7fffffffLL))
    return fail(DSA_EINVAL, "%s: k_cache needs k_num_pages >= 1 (got %lld)", fn,
                (long long)a->k_num_pages);
  if (prepared && (a->k_planes_capacity < a->num_positions || a->k_planes_capacity > 0x7fffffffLL ||
                   !aligned(a->k_planes, 256)))
    return fail(DSA_EINVAL, "%s: k_planes must be 256-byte aligned and laid out for at least "
                "num_positions = %lld positions (k_planes_capacity %lld)", fn,
                (long long)a->num_positions, (long long)a->k_planes_capacity);
  const dsa::IndexerWorkspace lay = dsa::indexer_workspace_layout(
      a->num_tokens, a->num_heads, a->num_positions, a->scores_out == nullptr, !prepared);
  if (lay.total > 0 && (!a->workspace || a->workspace_bytes < lay.total || !aligned(a->workspace, 256)))
    return fail(DSA_EWORKSPACE, "%s: workspace of %zu bytes (256-byte aligned) needed, got %zu",
                fn, lay.total, a->workspace ? a->workspace_bytes : (size_t)0);

  dsa::IndexerParams p = {};
  p.q = a->q_idx;
  p.k = a->k_idx;
  p.k_scale = a->k_scale;
  p.w = a->weights;
  p.limit = a->causal_limit;
  p.T = (int32_t)a->num_tokens;
  p.Hi = (int32_t)a->num_heads;
  p.S = (int32_t)a->num_positions;
  p.topk = (int32_t)a->topk;
  p.block_table = a->block_table;
  p.bt_stride = a->block_table_stride;
  p.page_size = (int32_t)(a->block_table ? a->page_size : 1);
  p.out = a->out;
  char *ws = static_cast<char *>(a->workspace);
  if (prepared) {
    const dsa::KPlanesLayout kl = dsa::k_planes_layout(a->k_planes_capacity);
    char *kp = static_cast<char *>(const_cast<void *>(a->k_planes));
    p.k_pieces = reinterpret_cast<int8_t *>(kp + kl.k_pieces);
    p.k_max = reinterpret_cast<int32_t *>(kp + kl.k_max);
    p.k_cs = reinterpret_cast<float *>(kp + kl.k_cs);
    p.k = nullptr;
    p.k_scale = nullptr;
    p.k_block0 = p.k_blocks = 0;
  } else {
    p.k_pieces = reinterpret_cast<int8_t *>(ws + lay.k_pieces);
    p.k_max = reinterpret_cast<int32_t *>(ws + lay.k_max);
    p.k_cs = reinterpret_cast<float *>(ws + lay.k_cs);
    p.k_block0 = 0;
    p.k_blocks = (int32_t)((a->num_positions + 15) / 16);
  }
  if (paged) {
    p.k_cache = a->k_cache;
    p.k_pages = a->k_pages;
    p.k_page_size = (int32_t)a->k_page_size;
    p.k_num_pages = (int32_t)a->k_num_pages;
  }
  p.scores = a->scores_out ? a->scores_out : reinterpret_cast<float *>(ws + lay.scores);
  const hipError_t e = dsa::launch_indexer(p, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(DSA_ELAUNCH, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return ok();
}

int dsa_indexer_prepare_k(const dsa_indexer_k_prepare_args *a, void *stream) {
  const char *fn = "dsa_indexer_prepare_k";
  if (!a) return fail(DSA_EINVAL, "%s: args is NULL", fn);
  if (a->num_positions < 0 || a->num_positions > 0x7fffffffLL || a->first_position < 0 ||
      a->count < 0)
    return fail(DSA_EINVAL, "%s: negative size or position", fn);
  if (a->k_planes_capacity < a->num_positions || a->k_planes_capacity > 0x7fffffffLL)
    return fail(DSA_EINVAL, "%s: k_planes_capacity %lld is below num_positions %lld", fn,
                (long long)a->k_planes_capacity, (long long)a->num_positions);
  if (a->first_position > a->num_positions || a->count > a->num_positions - a->first_position)
    return fail(DSA_EINVAL, "%s: positions [%lld, %lld) lie outside the %lld positions", fn,
                (long long)a->first_position, (long long)(a->first_position + a->count),
                (long long)a->num_positions);
  if (a->count == 0) return ok();
  if (!a->k_planes || !aligned(a->k_planes, 256))
    return fail(DSA_EINVAL, "%s: k_planes must be a 256-byte aligned buffer", fn);
  const bool paged = a->k_cache != nullptr;
  if (paged && (a->k_idx || a->k_scale))
    return fail(DSA_EINVAL, "%s: give k_idx/k_scale or k_cache, not both", fn);
  if (paged && (!a->k_pages || a->k_page_size <= 0 || a->k_page_size % 4 != 0 ||
                a->k_page_size > (1 << 24) || a->k_num_pages <= 0 ||
                a->k_num_pages > 0x7fffffffLL))
    return fail(DSA_EINVAL, "%s: k_cache needs k_pages, a k_page_size that is a positive multiple "
                "of 4 and k_num_pages >= 1", fn);
  if (!paged && (!a->k_idx || !a->k_scale)) return fail(DSA_EINVAL, "%s: NULL tensor pointer", fn);
  if (!aligned(a->k_idx, 16) || !aligned(a->k_scale, 4) || !aligned(a->k_cache, 16) ||
      !aligned(a->k_pages, 4))
    return fail(DSA_EINVAL, "%s: misaligned pointer (e4m3 rows need 16 bytes)", fn);
  const dsa::KPlanesLayout kl = dsa::k_planes_layout(a->k_planes_capacity);
  char *kp = static_cast<char *>(a->k_planes);
  dsa::IndexerParams p = {};
  p.k = a->k_idx;
  p.k_scale = a->k_scale;
  if (paged) {
    p.k_cache = a->k_cache;
    p.k_pages = a->k_pages;
    p.k_page_size = (int32_t)a->k_page_size;
    p.k_num_pages = (int32_t)a->k_num_pages;
  }
  p.S = (int32_t)a->num_positions;
  p.Hi = 16;
  p.k_pieces = reinterpret_cast<int8_t *>(kp + kl.k_pieces);
  p.k_max = reinterpret_cast<int32_t *>(kp + kl.k_max);
  p.k_cs = reinterpret_cast<float *>(kp + kl.k_cs);
  const int64_t b0 = a->first_position / 16, b1 = (a->first_position + a->count + 15) / 16;
  p.k_block0 = (int32_t)b0;
  p.k_blocks = (int32_t)(b1 - b0);
  const hipError_t e = dsa::launch_indexer_prepare_k(p, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(DSA_ELAUNCH, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return ok();
}

int dsa_indexer_k_append(const dsa_k_append_args *a, void *stream) {
  const char *fn = "dsa_indexer_k_append";
  if (!a) return fail(DSA_EINVAL, "%s: args is NULL", fn);
  if (a->num_tokens < 0 || a->num_pages < 0 || a->page_size <= 0 || a->page_size % 4 != 0)
    return fail(DSA_EINVAL, "%s: need num_tokens, num_pages >= 0 and a page_size that is a "
                "positive multiple of 4 (got %lld, %lld, %lld)", fn, (long long)a->num_tokens,
                (long long)a->num_pages, (long long)a->page_size);
  if (a->num_tokens > 0x7fffffffLL || a->num_pages * a->page_size > 0x7fffffffLL)
    return fail(DSA_EUNSUPPORTED, "%s: size beyond the supported range", fn);
  if (a->num_tokens == 0) return ok();
  if (!a->k || !a->slots || !a->k_cache) return fail(DSA_EINVAL, "%s: NULL tensor pointer", fn);
  if (a->k_stride < kIndexerHeadDim || (a->k_stride * 2) % 16 != 0 || !aligned(a->k, 16) ||
      !aligned(a->slots, 4) || !aligned(a->k_cache, 16))
    return fail(DSA_EINVAL, "%s: rows and k_cache must be 16-byte aligned (stride >= 128)", fn);
  dsa::KAppendParams p = {};
  p.k = static_cast<const uint16_t *>(a->k);
  p.k_stride = a->k_stride;
  p.slots = a->slots;
  p.n = (int32_t)a->num_tokens;
  p.cache = a->k_cache;
  p.num_slots = a->num_pages * a->page_size;
  p.page_size = (int32_t)a->page_size;
  const hipError_t e = dsa::launch_k_append(p, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(DSA_ELAUNCH, "%s: launch failed: %s", fn, hipGetErrorString(e));
  return ok();
}

}  // extern "C"
