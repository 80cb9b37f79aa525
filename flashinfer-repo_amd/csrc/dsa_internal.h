// dsa_internal.h -- shared declarations between the C-ABI layer and the HIP
// kernels of libdsa_amd.so (not part of the public ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dsa {

// MI355X (gfx950): 256 compute units in 8 XCDs.  The automatic split count is
// derived from this constant so that the workspace size a caller queries on
// the host without a device agrees with what the launch uses.
constexpr int kNumCU = 256;

constexpr int kHeadDimCkv = 512;
constexpr int kHeadDimKpe = 64;
constexpr int kHeadsPerGroup = 16;  // MFMA N dimension: one 16-head group
constexpr int kKeysPerTile = 32;       // keys gathered into one LDS ring stage
constexpr int kMinTilesPerSplit = 4;   // automatic splits keep >= 4 tiles of work each
constexpr int kMaxChunk = 1024;        // slot ids the multi-slice layouts keep in LDS (a ring)
constexpr int kMaxChunkWide = 2048;    // top-k entries one workgroup handles

struct AttnParams {
  const char *q_nope;  // byte strides below
  int64_t qn_st, qn_sh;
  const char *q_pe;
  int64_t qp_st, qp_sh;
  const char *ckv;
  int64_t ckv_sp, ckv_so;
  const char *kpe;
  int64_t kpe_sp, kpe_so;
  const int32_t *idx;  // element stride
  int64_t idx_st;
  char *out;
  int64_t out_st, out_sh;
  float *lse;  // element strides
  int64_t lse_st, lse_sh;
  int32_t T, H, K, page_size;
  int64_t num_slots;
  // slot / page_size = (slot * ps_magic) >> (31 + ps_shift) for every slot
  // below 2^31 (round-up reciprocal: ps_shift = ceil(log2 page_size),
  // ps_magic = floor(2^(31 + ps_shift) / page_size) + 1 < 2^32)
  uint32_t ps_magic;
  int32_t ps_shift;
  float scale_log2;  // sm_scale * log2(e)
  int32_t num_splits, chunk;
  // Unnormalised partial outputs and (reference max in log2 units, sum):
  // for the merge kernel [T][S][H][512] and [T][S][H][2]; for the in-kernel
  // merge the same part_acc space in per-wave lane-order regions and 16
  // pairs per wave in part_ml (room for [T][S][H][16] floats).
  float *part_acc;
  float *part_ml;
  int32_t partial_only;  // write partials even when num_splits == 1
  // Split merge inside the attention kernel: per-wave arrival counters
  // [T][head blocks][8], zero before the launch and left zero by it.  Null:
  // the separate merge kernel runs.
  uint32_t *counters;
  // Narrow addressing (set when the host has checked it applies): slot s's
  // rows sit at byte s * ckv_rs / s * kpe_rs of their caches, every such
  // offset of a valid slot lies below ckv_extent / kpe_extent <= 2^31, and
  // ckv_rs, kpe_rs and the slot count are below 2^24 (24-bit multiplies).
  int32_t narrow;
  uint32_t ckv_rs, kpe_rs, ckv_extent, kpe_extent;
};

// Counter words a split call with in-kernel merge uses.
inline int64_t attn_counter_words(int64_t T, int head_blocks) { return T * head_blocks * 8; }

// Workgroups per token along the head axis (each covers up to 8 groups of 16).
int attn_head_blocks(int H);
// Longest top-k chunk one workgroup of the layout for H heads handles.
int attn_max_chunk(int H);
// Whether split calls with counters merge inside the attention kernel for H
// heads and S splits: the four-wave layout of an odd number of head groups,
// up to kMaxInKernelMergeSplits splits (the last chunk's wave reads every
// chunk's partial; from 5 splits on the merge kernel, which spreads that
// work over the tokens and heads, is faster: H=16 top-k 2048, 8 splits, T=1
// 16.3 against 14.5 us, T=32 22.6 against 21.7 us; at 4 splits the in-kernel
// merge is as fast or faster and saves a launch).  Otherwise the merge kernel
// runs and the counters are not touched.
constexpr int kMaxInKernelMergeSplits = 4;
bool attn_merges_in_kernel(int H, int64_t S);
// Whether a call of T tokens, H heads and S splits runs the four-wave layout
// (one workgroup per 16-head group and chunk): always for an odd number of
// head groups, for an even one while its T * S * groups workgroups fit the
// CUs in one round.
bool attn_wave_layout(int64_t T, int H, int64_t S);

// Whole call: per-chunk attention, then (num_splits > 1) the merge.
hipError_t launch_attention(const AttnParams &p, hipStream_t stream);
// The two halves on their own: with num_splits > 1 the first writes only the
// partials; the second merges part_acc/part_ml into out/lse.
hipError_t launch_attention_partial(const AttnParams &p, hipStream_t stream);
hipError_t launch_attention_merge(const AttnParams &p, hipStream_t stream);

}  // namespace dsa

struct dsa_attn_args;

namespace dsa {

// dsa_attn_fwd's validation and launch, for entry points that share it (fn
// names the entry point in error messages).
int attn_fwd(const char *fn, const dsa_attn_args *a, void *stream);
// Sets the thread-local error string; returns code.
int set_error(int code, const char *msg);
// Workspace a split call of this shape needs (0 without a split).
size_t attn_split_workspace(int64_t T, int64_t H, int64_t K, int32_t requested);

// Lightning indexer.  Workspace layout (see indexer_workspace_layout):
//   k_pieces [ceil(S/16)][3 pieces][2 k-steps][1024 B]  MFMA B operands, lane order
//   k_max    [ceil(S/16)]                               max |value * 2^9| per block
//   k_cs     [S] fp32                                   c_s = fl32(k_scale * 2^-18) per position
//   scores   [T][S] fp32                                (unless the caller's)
struct IndexerParams {
  const uint8_t *q;       // [T][Hi][128] e4m3 codes
  const uint8_t *k;       // [S][128] e4m3 codes (or null: paged cache below)
  const float *k_scale;   // [S] (null with a paged cache)
  // paged K cache: position s is token s % k_page_size of page k_pages[s /
  // k_page_size]; codes at page*k_page_size*132 + off*128, the fp32 scale at
  // page*k_page_size*132 + k_page_size*128 + off*4
  const uint8_t *k_cache;
  const int32_t *k_pages;
  int32_t k_page_size;
  int32_t k_num_pages;    // page ids outside [0, k_num_pages) read as zero rows
  float *k_cs;            // [S] workspace: c_s = fl32(k_scale * 2^-18), written by the prep kernel
  const float *w;         // [T][Hi]
  const int32_t *limit;   // [T]
  int32_t T, Hi, S, topk;
  const int32_t *block_table;
  int64_t bt_stride;
  int32_t page_size;
  int32_t *out;           // [T][topk]
  float *scores;          // [T][S] (workspace or caller buffer)
  int8_t *k_pieces;
  int32_t *k_max;
  int32_t blocks_per_wg;  // 16-position blocks one score workgroup walks (set by the launcher)
  // k blocks the prep kernel derives planes for: [k_block0, k_block0 + k_blocks)
  // (0 blocks when the call reads prepared K planes)
  int32_t k_block0, k_blocks;
};

struct IndexerWorkspace {
  size_t k_pieces, k_max, k_cs, scores, total;  // byte offsets; total = size
};

// Offsets of the indexer's workspace regions; scores are left out when the
// caller provides the score buffer, the k regions when the call reads
// prepared K planes.
IndexerWorkspace indexer_workspace_layout(int64_t T, int64_t Hi, int64_t S, bool own_scores,
                                          bool own_k);

hipError_t launch_indexer(const IndexerParams &p, hipStream_t stream);
// Only the k planes of blocks [k_block0, k_block0 + k_blocks) (K preparation).
hipError_t launch_indexer_prepare_k(const IndexerParams &p, hipStream_t stream);

// Prepared K planes (dsa_indexer_prepare_k): the K half of the workspace
// layout, [k_pieces][k_max][k_cs] of S positions, 256-byte aligned regions.
struct KPlanesLayout {
  size_t k_pieces, k_max, k_cs, total;
};
KPlanesLayout k_planes_layout(int64_t S);

// Quantise-on-append into the paged indexer K cache (layout above).
struct KAppendParams {
  const uint16_t *k;  // [n][k_stride] bf16 bits
  int64_t k_stride;
  const int32_t *slots;
  int32_t n;
  uint8_t *cache;
  int64_t num_slots;
  int32_t page_size;
};
hipError_t launch_k_append(const KAppendParams &p, hipStream_t stream);

}  // namespace dsa
