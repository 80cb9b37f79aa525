// dsa_attention.hip -- gather-fused sparse MLA attention for gfx950 (CDNA4).
//
// Computes, per token t and head h (semantics of the reference's golden
// run(), solution/triton/indexer_kernel.py:436-497, and of its Triton kernels
// solution/triton/kernel.py:9-136 / :343-434 / :437-493):
//
//   x_j   = (q_nope[t,h] . ckv[s_j] + q_pe[t,h] . kpe[s_j]) * sm_scale
//   out   = sum_j softmax(x)_j * ckv[s_j]              (bf16)
//   lse   = logsumexp(x) / ln 2                        (fp32, base 2)
//
// over the valid slots s_j of sparse_indices[t] (-1 = padding).
//
// Work decomposition.  One workgroup = one (token, top-k chunk, block of
// head groups).  Its waves share a 4-stage LDS ring of 32-key tiles (the
// whole 160 KB of LDS): every tile is gathered by LDS DMA (16 B per lane
// straight into LDS, no VGPR staging; one 1 KB ckv row per instruction, 8 kpe
// rows per instruction), two tiles in flight while two are in use.  The
// chunk's slot ids are staged in LDS (4 bytes per key, so no index load sits
// in front of a gather) and the valid-key mask of every tile is kept in one
// VGPR (lane i: tile i).  Padding keys gather a zero row, which keeps the
// number of loads per wave and tile fixed and makes the vmcnt-based stage
// waits exact.  Dense caches
// below 2 GB (every BASELINE shape) are gathered with buffer_load ... lds at
// 32-bit offsets slot * row stride (one 24-bit multiply per key, one readlane
// per row); a padding key's offset lies past the buffer's range, and an
// out-of-range buffer load returns zeros, which the DMA writes as the row.
// Other caches take global_load_lds_dwordx4 at 64-bit addresses, the page
// division as a multiply by a host-computed reciprocal, and a zero row in
// global memory.
//
// Each wave belongs to one 16-head group and owns one slice of the 512 output
// features.  Per tile:
//   S^T[32 keys x 16 heads] = K[keys x 576] . Q^T       (bf16 MFMA 16x16x32)
//     -- when FS > 1 waves share a head group, they split the 2 key blocks x
//        576 features of this product into equal parts (QkSplit) and add the
//        partial S^T through LDS in a fixed order, so every wave of the group
//        holds identical scores;
//   online softmax in fp32 (log2 domain), with the reference max moved only
//   when scores overshoot it by more than kRescaleSlack;
//   O^T[slice x 16 heads] += V^T[slice x 32 keys] . P^T  (bf16 MFMA 16x16x32,
//     P split into bf16 hi + lo parts, ~16-bit P; the V^T operand is read
//     with ds_read_b64_tr_b16, which transposes 16-bit elements across lanes).
// Computing S^T (keys as the MFMA M dimension) leaves P^T in exactly the lane
// layout the PV product takes as its B operand.
//
// Splits.  With one chunk per token the workgroup writes the bf16 output and
// lse directly.  Otherwise each workgroup writes an unnormalised fp32 partial
// (acc, m, l) and the partials of a token are merged with log-sum-exp
// weights in split order (reference merge algebra: kernel.py:461-493, -inf
// guards :475-476), so results are deterministic: in the 8-slice layout
// inside this kernel by the wave that finishes a feature slice last (device-
// coherent sc1 stores and loads plus a per-wave arrival counter, no L2
// write-back), otherwise by dsa_attn_combine_kernel.  Both give the same
// bits.
//
// MFMA 16x16x32 bf16 lane layout used throughout (lane = 16*g + r):
//   A (16 x 32): lane holds row r, k-slots 8g..8g+7
//   B (32 x 16): lane holds column r, k-slots 8g..8g+7
//   D (16 x 16): lane holds column r, rows 4g..4g+3
// Only the A/B k-slot assignment being identical matters for a product, so
// the kernel assigns k-slots to features or keys as convenient.
//
// Within a 16-key block, MFMA row m of S^T holds key pi(m) = 8*((m>>2)&1) +
// (m>>3) + 2*(m&3), so lane group g owns keys kbase(g) + {0,2,4,6} with
// kbase = 0, 8, 1, 9.  The QK operand reads still touch 16 distinct rows
// (conflict-free with the 1040-byte pitch), and the PV transpose reads of one
// 32-lane half touch 8 rows whose 32-byte pieces land on 8 disjoint bank
// ranges, which is conflict-free too.
//
// ds_read_b64_tr_b16, per 16-lane group: lane i receives element i%4 of the
// 4-element (8-byte) rows addressed by lanes 4j + i/4, j = 0..3.  Pointing
// lanes 4j..4j+3 at 8-byte pieces f0..f0+15 of key row j gives lane i the
// feature f0+i of keys 0..3: one half of an A operand of V^T.
#include "dsa_internal.h"

namespace dsa {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

// Raw buffer resources (stride 0, byte-sized range, 32-bit data format) and
// the sc1 cache policy bit of buffer loads and stores (device coherence).
constexpr int kBufferFlags = 0x00020000;
constexpr int kSC1 = 16;

// LDS geometry (bytes).  A ckv row is padded from 1024 to 1040 B so the 16
// rows one MFMA operand read touches fall in distinct banks; kpe rows are
// gathered 8 per DMA instruction in chunk-major order (lane i of the DMA holds
// 16-byte chunk i/8 of row i%8), so a column read of 16 rows hits 16
// consecutive chunks.
constexpr int kCkvPitch = 1024 + 16;
constexpr int kKpeGroupPitch = 1024 + 128;
constexpr int kCkvStageBytes = kKeysPerTile * kCkvPitch;
constexpr int kStageBytes = kCkvStageBytes + (kKeysPerTile / 8) * kKpeGroupPitch;
constexpr int kStages = 4;
// After the ring: slot ids (4 bytes per key) and, for layouts whose waves
// share a head group, the partial-score exchange (one f32x4 per lane per
// wave).  One-slice layouts exchange nothing and stage the ids of a whole
// 2048-key chunk; the others keep a ring of 32 tiles' ids, refilled half by
// half while the chunk runs (refill_ids in the kernel).
template <int FS>
struct Lds {
  static constexpr int kMaxChunkKeys = kMaxChunkWide;
  static constexpr int kSlotIds = FS == 1 ? kMaxChunkWide : kMaxChunk;
  static constexpr int kRingTiles = kSlotIds / kKeysPerTile;
  static constexpr int kSlotBytes = kSlotIds * 4;
  static constexpr int kXchgBytes = FS == 1 ? 0 : 8 * 64 * 16;
  static constexpr int kBytes = kStages * kStageBytes + kSlotBytes + kXchgBytes;
  static_assert(kBytes <= 160 * 1024, "LDS budget of one gfx950 CU");
  static_assert(kMaxChunkKeys / kKeysPerTile <= 64, "one mask lane per tile");
  static_assert(kRingTiles % 32 == 0, "refills are halves of 16 tiles");
};

// The running max is only moved (and the accumulator rescaled) when a head's
// scores exceed it by more than this many log2 units, so probabilities stay
// below 2^8 and most tiles skip the rescale entirely.
constexpr float kRescaleSlack = 8.0f;

// Padding keys gather from here (global memory, never written).
__device__ __attribute__((aligned(64))) const uint4 g_zero_row[64] = {};
// Slot-id refills read keys past the chunk from here: -1, padding.
__device__ __attribute__((aligned(64))) const int32_t g_minus_one[64] = {
    -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1,
    -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1,
    -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1, -1};

__device__ __forceinline__ void lds_dma16(const void *gsrc, void *ldst) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)gsrc,
                                   (__attribute__((address_space(3))) void *)ldst, 16, 0, 0);
}

// 16 bytes per lane from a buffer resource at byte offset voff (lane i lands
// at ldst + 16 i; an offset past the resource's range lands zeros).
__device__ __forceinline__ void lds_dma16_buf(__amdgpu_buffer_rsrc_t rsrc, void *ldst, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void *)ldst, 16,
                                           voff, 0, 0, 0);
}

// 4 bytes per lane: lane i lands at ldst + 4 i.
__device__ __forceinline__ void lds_dma4(const void *gsrc, void *ldst) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)gsrc,
                                   (__attribute__((address_space(3))) void *)ldst, 4, 0, 0);
}

// V^T operands of four feature blocks F0 .. F0+3 with ds_read_b64_tr_b16: for
// block f, keys 0-15 at vsrc + 32 f and keys 16-31 one 16-row block further
// (ROWB bytes).  The eight reads and their lgkmcnt(0) wait are one asm
// statement, so the compiler neither touches the destinations before the data
// lands nor inserts the vmcnt(0) it puts in front of the builtin form (it
// cannot tell the transpose read from an access to the LDS DMA targets).
template <int F0, int ROWB>
__device__ __forceinline__ void tr_read4(const char *vsrc, bf16x8 (&av)[4]) {
  const uint32_t va = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char *)vsrc;
  u32x2 a0, a1, a2, a3, b0, b1, b2, b3;
  asm volatile(
      "ds_read_b64_tr_b16 %0, %8 offset:%9\n\t"
      "ds_read_b64_tr_b16 %4, %8 offset:%13\n\t"
      "ds_read_b64_tr_b16 %1, %8 offset:%10\n\t"
      "ds_read_b64_tr_b16 %5, %8 offset:%14\n\t"
      "ds_read_b64_tr_b16 %2, %8 offset:%11\n\t"
      "ds_read_b64_tr_b16 %6, %8 offset:%15\n\t"
      "ds_read_b64_tr_b16 %3, %8 offset:%12\n\t"
      "ds_read_b64_tr_b16 %7, %8 offset:%16\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(a0), "=&v"(a1), "=&v"(a2), "=&v"(a3), "=&v"(b0), "=&v"(b1), "=&v"(b2), "=&v"(b3)
      : "v"(va), "i"(F0 * 32), "i"(F0 * 32 + 32), "i"(F0 * 32 + 64), "i"(F0 * 32 + 96),
        "i"(ROWB + F0 * 32), "i"(ROWB + F0 * 32 + 32), "i"(ROWB + F0 * 32 + 64),
        "i"(ROWB + F0 * 32 + 96)
      : "memory");
  av[0] = __builtin_bit_cast(bf16x8, (u32x4){a0[0], a0[1], b0[0], b0[1]});
  av[1] = __builtin_bit_cast(bf16x8, (u32x4){a1[0], a1[1], b1[0], b1[1]});
  av[2] = __builtin_bit_cast(bf16x8, (u32x4){a2[0], a2[1], b2[0], b2[1]});
  av[3] = __builtin_bit_cast(bf16x8, (u32x4){a3[0], a3[1], b3[0], b3[1]});
}

// tr_read4 for every feature block of a wave's slice, four at a time, each
// batch followed by its MFMAs (fn(f0, av)).
template <int NFB, int ROWB, int F0 = 0, typename Fn>
__device__ __forceinline__ void for_tr_batches(const char *vsrc, Fn &&fn) {
  static_assert(NFB % 4 == 0, "feature blocks come in batches of four");
  if constexpr (F0 < NFB) {
    bf16x8 av[4];
    tr_read4<F0, ROWB>(vsrc, av);
    fn(F0, av);
    for_tr_batches<NFB, ROWB, F0 + 4>(vsrc, fn);
  }
}

__device__ __forceinline__ uint64_t readlane64(uint64_t v, int lane) {
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, lane);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), lane);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Key (within a 16-key block) that MFMA row m of S^T stands for.
__device__ __forceinline__ int key_of_row(int m) {
  return ((m >> 2) & 1) * 8 + (m >> 3) + 2 * (m & 3);
}

// Waits until at most N of this wave's vector-memory operations are
// outstanding (they complete in issue order).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// QK split among the NP waves that share a key block: part p takes the
// 32-feature nope steps [16p/NP, 16(p+1)/NP) and the kpe features
// [64p/NP, 64(p+1)/NP) -- NP = 1: 16 nope + two 32-feature kpe steps; NP = 2:
// 8 + one; NP = 4: 4 nope steps + one 16-feature kpe step (the 16x16x16 MFMA).
// Every part has the same shape, so a wave's range is an address offset.
template <int NP>
struct QkSplit {
  static_assert(NP == 1 || NP == 2 || NP == 4, "parts per key block");
  static constexpr int kNope = 16 / NP;               // 32-feature nope steps per part
  static constexpr int kPe32 = NP <= 2 ? 2 / NP : 0;  // 32-feature kpe steps per part
  static constexpr bool kPe16 = NP == 4;              // one 16-feature kpe step
};

// Q^T operands (the B side of S^T = K Q^T) of one part, this lane's k-slots.
template <int NP>
struct QkOperands {
  bf16x8 nope[QkSplit<NP>::kNope];
  bf16x8 pe32[QkSplit<NP>::kPe32 > 0 ? QkSplit<NP>::kPe32 : 1];
  i16x4 pe16;
};

// Partial S^T of part `part` for this lane's key: rowp = its ckv row in LDS
// (+ 16 g), kp = its kpe row's first chunk (kpe rows are chunk-major: chunk c
// of row r at (8c + r) * 16 within the 8-row group).  Split parts keep two
// independent MFMA chains added at the end; the full range of the one-slice
// layouts keeps one chain (its waves have no registers to spare).
template <int NP>
__device__ __forceinline__ f32x4 qk_part(int part, const char *rowp, const char *kp,
                                         const QkOperands<NP> &q, int g) {
  using Q = QkSplit<NP>;
  constexpr int kChains = NP > 1 ? 2 : 1;
  f32x4 c[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  const char *np = rowp + part * (Q::kNope * 64);
#pragma unroll
  for (int k = 0; k < Q::kNope; ++k)
    c[k % kChains] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const bf16x8 *)(np + k * 64),
                                                             q.nope[k], c[k % kChains], 0, 0, 0);
#pragma unroll
  for (int j = 0; j < Q::kPe32; ++j) {
    const int step = part * Q::kPe32 + j;  // 32 kpe features = chunks 4 step .. 4 step + 3
    c[(Q::kNope + j) % kChains] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
        *(const bf16x8 *)(kp + (step * 4 + g) * 128), q.pe32[j], c[(Q::kNope + j) % kChains], 0, 0, 0);
  }
  if constexpr (Q::kPe16) {
    // features 16 part + 4g .. +3: chunk 2 part + g/2, bytes (g & 1) * 8 of it
    const i16x4 a = *(const i16x4 *)(kp + (2 * part + (g >> 1)) * 128 + (g & 1) * 8);
    c[1] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, q.pe16, c[1], 0, 0, 0);
  }
  return kChains == 2 ? c[0] + c[1] : c[0];
}

// Source of one wave's share of a tile gather (see tile_src in the kernel).
template <int ROWS>
struct GatherSrc {
  uint32_t row[ROWS];  // narrow: ckv byte offset of each row this wave gathers
  uint32_t ko;         // narrow: kpe byte offset of this lane's 16-byte chunk
  uint64_t ckv, kpe;   // otherwise: row addresses of this lane's key
};

// W waves per workgroup; FS waves share one 16-head group, each owning
// 512/FS output features.  W/FS head groups per workgroup.  With FS > 1 the
// waves of a group split S^T = K Q^T into 2 key blocks x kParts step ranges.
template <int W, int FS>
struct Ring {
  static constexpr int kHG = W / FS;
  static constexpr int kNFB = 32 / FS;            // 16-feature blocks per wave
  static constexpr int kRows = kKeysPerTile / W;  // ckv rows one wave gathers per tile
  static constexpr int kLoads = kRows + 1;        // + one kpe DMA (full or half)
  static constexpr int kParts = FS >= 2 ? FS / 2 : 1;  // QK parts per key block (QkSplit)
  static constexpr int kBlocks = FS >= 2 ? 1 : 2;      // key blocks one wave computes
  static_assert(W == 4 || W == 8, "gather split assumes 4 or 8 waves");
  static_assert(FS == 1 || FS == 2 || FS == 4 || FS == 8, "feature slices");
};

// NARROW: the caches are dense (slot s at byte s * row stride) and below
// 2 GB, so the gathers address them with 32-bit offsets through buffer
// resources; otherwise through 64-bit addresses with the page arithmetic.
template <int W, int FS, bool NARROW>
__global__ __launch_bounds__(W * 64, 1) void dsa_attn_ring_kernel(AttnParams p) {
  using R = Ring<W, FS>;
  using L = Lds<FS>;
  __shared__ __attribute__((aligned(16))) char lds[L::kBytes];
  int32_t *slots = (int32_t *)(lds + kStages * kStageBytes);  // -1: padding / invalid
  f32x4 *xbuf = (f32x4 *)(lds + kStages * kStageBytes + L::kSlotBytes);  // FS > 1 only

  const int t = blockIdx.x / p.num_splits;
  const int split = blockIdx.x - t * p.num_splits;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int hg = wave / FS;
  const int fs = wave - hg * FS;
  const int head = (blockIdx.y * R::kHG + hg) * kHeadsPerGroup + r16;
  // this wave's share of S^T: key block qb0 (+1 if kBlocks == 2), step range part
  const int qb0 = FS >= 2 ? (fs & 1) : 0;
  const int part = FS >= 2 ? (fs >> 1) : 0;

  // the 8-slice layout shares the softmax work through LDS (softmax_publish /
  // consume_words)
  constexpr bool kShared = W == 8 && FS == 8;
  const int k_begin = split * p.chunk;
  const int n_keys = max(0, min(p.K, k_begin + p.chunk) - k_begin);
  const int n_tiles = (n_keys + kKeysPerTile - 1) / kKeysPerTile;

  // Q^T as the B operand of S^T = K Q^T (QkSplit: this wave's part of the
  // 576 features; per 32-feature step the lane holds features 8g..8g+7).
  // Issued before the slot-id staging, whose LDS stores wait for the index
  // loads: both loads are then in flight together (one memory latency).
  QkOperands<R::kParts> qreg;
  {
    using Q = QkSplit<R::kParts>;
    const char *qn = p.q_nope + t * p.qn_st + head * p.qn_sh + g * 16 + part * (Q::kNope * 64);
    const char *qp = p.q_pe + t * p.qp_st + head * p.qp_sh;
#pragma unroll
    for (int k = 0; k < Q::kNope; ++k) qreg.nope[k] = *(const bf16x8 *)(qn + k * 64);
#pragma unroll
    for (int j = 0; j < Q::kPe32; ++j)
      qreg.pe32[j] = *(const bf16x8 *)(qp + (part * Q::kPe32 + j) * 64 + g * 16);
    if constexpr (Q::kPe16) qreg.pe16 = *(const i16x4 *)(qp + part * 32 + g * 8);
  }
  // ---- stage the slot ids of the chunk's first kRingTiles tiles (padding and
  // out-of-range ids -> -1); all index loads are issued before the first
  // store so they overlap
  {
    constexpr int kPer = L::kSlotIds / (W * 64);
    const int32_t *src = p.idx + (int64_t)t * p.idx_st + k_begin;
    int sv[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = threadIdx.x + k * W * 64;
      sv[k] = i < n_keys ? src[i] : -1;
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = threadIdx.x + k * W * 64;
      const int s = sv[k];
      const bool valid = s >= 0 && (int64_t)s < p.num_slots;
      if (i < n_tiles * kKeysPerTile) slots[i] = valid ? s : -1;
    }
  }

  // Retire the Q loads with a wait the compiler sees (s_waitcnt vmcnt(0)), so
  // its own bookkeeping has nothing outstanding when the gather ring starts
  // and it adds no drain at the loop header.
  __builtin_amdgcn_s_waitcnt(0x0F70);
  __syncthreads();  // slot ids visible; nothing gathered yet


  // ---- gather issue: this wave's share of tile j into stage j % kStages.
  // Lane l owns key 8*grp + (l & 7) of the tile, grp being the kpe group
  // (8 rows) this wave gathers (a half group when W == 8).
  const int grp = (W == 4) ? wave : (wave >> 1);
  const int row0 = (W == 4) ? 0 : 4 * (wave & 1);  // first ckv row within the group
  // valid-key mask of tile i in lane i (wave-uniform reads with readlane):
  // tiles of the first ring pass are masked after the first gathers are
  // issued, tiles of refilled ids when they are issued
  uint32_t tile_masks = 0;
  const bool kpe_lane = W == 4 || (lane >> 5) == (wave & 1);  // this lane's kpe chunk is gathered here
  auto note_refilled_mask = [&](int j, const int32_t *ids) {
    if (FS >= 2 && j >= L::kRingTiles) {
      const uint32_t id = (uint32_t)ids[lane & 31];
      const uint32_t bits = (uint32_t)__ballot(id < (uint32_t)p.num_slots);
      tile_masks = lane == j ? bits : tile_masks;
    }
  };
  // NARROW: one 32-bit byte offset per key (slot * row stride); a padding or
  // out-of-range key gets kOOB, past the end of every buffer, and a buffer
  // load beyond its range returns zeros, so its row lands as zeros.
  constexpr uint32_t kOOB = 0x80000000u;
  const auto ckv_rsrc = __builtin_amdgcn_make_buffer_rsrc((void *)p.ckv, 0, (int)p.ckv_extent, kBufferFlags);
  const auto kpe_rsrc = __builtin_amdgcn_make_buffer_rsrc((void *)p.kpe, 0, (int)p.kpe_extent, kBufferFlags);
  // A tile's gather in two steps: tile_src reads the slot ids and computes the
  // row addresses (LDS reads and arithmetic, done before the barrier that
  // frees the stage, off the path between the barriers); fire_tile issues the
  // DMAs into stage j % kStages.
  using TileSrc = GatherSrc<R::kRows>;
  auto tile_src = [&](int j) {
    TileSrc a;
    const int32_t *ids = slots + (j % L::kRingTiles) * kKeysPerTile;  // refilled ids are raw
    note_refilled_mask(j, ids);
    if constexpr (NARROW) {
      const uint32_t sl = (uint32_t)ids[grp * 8 + (lane & 7)];
      const bool ok = sl < (uint32_t)p.num_slots;  // -1 wraps to 2^32 - 1
      const uint32_t co = ok ? __umul24(sl, p.ckv_rs) : kOOB;
#pragma unroll
      for (int m = 0; m < R::kRows; ++m) a.row[m] = __builtin_amdgcn_readlane(co, row0 + m);
      a.ko = (ok ? __umul24(sl, p.kpe_rs) : kOOB) + (lane >> 3) * 16;
    } else {
      const int sl = ids[grp * 8 + (lane & 7)];
      a.ckv = a.kpe = (uint64_t)(const char *)g_zero_row;
      if (sl >= 0 && (int64_t)sl < p.num_slots) {
        const uint32_t pg = (uint32_t)(((uint64_t)(uint32_t)sl * p.ps_magic) >> (31 + p.ps_shift));
        const uint32_t of = (uint32_t)sl - pg * (uint32_t)p.page_size;
        a.ckv = (uint64_t)(p.ckv + (int64_t)pg * p.ckv_sp + (int64_t)of * p.ckv_so);
        a.kpe = (uint64_t)(p.kpe + (int64_t)pg * p.kpe_sp + (int64_t)of * p.kpe_so);
      }
    }
    return a;
  };
  auto fire_tile = [&](int j, const TileSrc &a) {
    char *st = lds + (j & (kStages - 1)) * kStageBytes;
    char *kdst = st + kCkvStageBytes + grp * kKpeGroupPitch;
    if constexpr (NARROW) {
#pragma unroll
      for (int m = 0; m < R::kRows; ++m)
        lds_dma16_buf(ckv_rsrc, st + (grp * 8 + row0 + m) * kCkvPitch, a.row[m] + lane * 16);
      if (kpe_lane) lds_dma16_buf(kpe_rsrc, kdst, a.ko);
    } else {
#pragma unroll
      for (int m = 0; m < R::kRows; ++m) {
        const char *src = (const char *)readlane64(a.ckv, row0 + m) + lane * 16;
        lds_dma16(src, st + (grp * 8 + row0 + m) * kCkvPitch);
      }
      if (kpe_lane) lds_dma16((const char *)a.kpe + (lane >> 3) * 16, kdst);
    }
  };

  f32x4 acc[R::kNFB];
#pragma unroll
  for (int i = 0; i < R::kNFB; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;  // reference max of x*log2(e) for this lane's head
  float l_run = 0.f;        // running sum over this lane's keys (reduced at the end)

  // ---- per-tile stages, shared by both loop shapes below
  // S^T partial (or, FS == 1, complete) of the wave's key blocks and k-steps
  auto scores = [&](const char *st_ckv, f32x4 (&sacc)[2]) {
    const char *st_kpe = st_ckv + kCkvStageBytes;
#pragma unroll
    for (int bb = 0; bb < R::kBlocks; ++bb) {
      const int b = qb0 + bb;
      const int kk = b * 16 + key_of_row(r16);
      const char *rowp = st_ckv + kk * kCkvPitch + g * 16;
      const char *kp = st_kpe + (kk >> 3) * kKpeGroupPitch + (kk & 7) * 16;
      sacc[bb] = qk_part<R::kParts>(part, rowp, kp, qreg, g);
    }
  };
  // Partial S^T exchange: slot w holds wave w's partial of its key block.
  // The 8-slice layout reads single components (value_logit), so it keeps
  // them component-major (each read is 64 consecutive words, no bank
  // conflicts); the others read whole f32x4 per lane.
  auto xput = [&](const f32x4 &v) {
    if constexpr (kShared) {
      float *x = (float *)xbuf;
#pragma unroll
      for (int k = 0; k < 4; ++k) x[(wave * 4 + k) * 64 + lane] = v[k];
    } else {
      xbuf[wave * 64 + lane] = v;
    }
  };
  auto xget = [&](int slot) -> f32x4 {
    if constexpr (kShared) {
      const float *x = (const float *)xbuf;
      return f32x4{x[(slot * 4 + 0) * 64 + lane], x[(slot * 4 + 1) * 64 + lane],
                   x[(slot * 4 + 2) * 64 + lane], x[(slot * 4 + 3) * 64 + lane]};
    } else {
      return xbuf[slot * 64 + lane];
    }
  };
  // the group's partial S^T, added in a fixed order (after the exchange)
  auto reduce = [&](f32x4 (&sacc)[2]) {
    const int base = hg * FS;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      f32x4 c = xget(base + b);
#pragma unroll
      for (int pp = 1; pp < R::kParts; ++pp) c += xget(base + b + 2 * pp);
      sacc[b] = c;
    }
  };
  const int kbase = (g & 1) * 8 + (g >> 1);
  // online softmax of one tile -> its probabilities (bf16 hi + lo parts)
  auto softmax = [&](const f32x4 (&sacc)[2], uint32_t vmask, bf16x8 &p_hi, bf16x8 &p_lo) {
    // ---- online softmax.  This lane: head r16; slot (b, k) holds key
    // b*16 + kbase + 2k.  d = x*log2(e) - m_run with the lazily moved
    // reference m_run; the tile max is only reduced when some score
    // overshoots the reference by more than the slack (always on the first
    // valid tile, where m_run = -inf).
    const uint32_t vm = vmask >> kbase;
    const bool full = vmask == 0xffffffffu;  // wave-uniform
    const float c = p.scale_log2;
    float d[8];
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float v = __builtin_fmaf(sacc[b][k], c, -m_run);
        d[b * 4 + k] = (full || ((vm >> (b * 16 + 2 * k)) & 1u)) ? v : -INFINITY;
      }
    bool over = false;
#pragma unroll
    for (int k = 0; k < 8; ++k) over |= d[k] > kRescaleSlack;
    if (__ballot(over) != 0) {  // wave-uniform
      float mx = -INFINITY;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int k = 0; k < 4; ++k)
          if (full || ((vm >> (b * 16 + 2 * k)) & 1u)) mx = fmaxf(mx, sacc[b][k] * c);
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run, mx);
      const float alpha = (m_run == -INFINITY) ? 0.f : fast_exp2(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int fb = 0; fb < R::kNFB; ++fb) acc[fb] *= alpha;
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const float v = __builtin_fmaf(sacc[b][k], c, -m_run);
          d[b * 4 + k] = (full || ((vm >> (b * 16 + 2 * k)) & 1u)) ? v : -INFINITY;
        }
    }
    // m_run stays -inf only while no valid key has been seen; then every
    // d is -inf and the probabilities are 0.
    float psum = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float pv = fast_exp2(d[k]);
      psum += pv;
      p_hi[k] = (__bf16)pv;
      p_lo[k] = (__bf16)(pv - (float)p_hi[k]);
    }
    l_run += psum;
  };
  // Probability exchange of the 8-slice layout (FS == 8, one head group):
  // value v = b*4 + k of every lane (head r16, key b*16 + kbase + 2k) is
  // computed by wave v alone and passed on through LDS, instead of every wave
  // reducing the partial scores and exponentiating all 512 values.  The words
  // live in the 128-byte padding after each kpe row group of the four stages,
  // which neither the gather nor the score reads touch: value v, lane l at
  // padding chunk 2v + l/32, word l%32.  A word is bf16 hi << 16 | bf16 lo; hi
  // is never negative, so its sign bit carries "this value overshoots the
  // reference max", and since every wave reads all 512 words they all take
  // the same (rare) rescale branch.
  auto pword = [&](int v, int l) -> uint32_t * {
    const int c = 2 * v + (l >> 5);
    return (uint32_t *)(lds + (c >> 2) * kStageBytes + kCkvStageBytes + (c & 3) * kKpeGroupPitch +
                        1024 + (l & 31) * 4);
  };
  // The words of tile i are published after the partial exchange of
  // iteration i and read after the first barrier of iteration i + 1 (which
  // also finds tile i + 1 landed), one barrier per tile for both.  This
  // wave's value waits in pv_pending until the words show whether the tile
  // overshot the reference max.
  float pv_pending = 0.f;
  auto publish = [&](float d, bool flag) {
    const float pv = fast_exp2(d);
    const __bf16 hi = (__bf16)pv;
    const __bf16 lo = (__bf16)(pv - (float)hi);
    const uint32_t w = ((uint32_t)__builtin_bit_cast(uint16_t, hi) | (flag ? 0x8000u : 0u)) << 16 |
                       (uint32_t)__builtin_bit_cast(uint16_t, lo);
    *pword(wave, lane) = w;
    pv_pending = pv;
  };
  // this lane's score of value v = wave (head r16, key b*16 + kbase + 2k):
  // the partials added in the order reduce() uses; -inf when masked
  auto value_logit = [&](uint32_t vmask) -> float {
    const int b = wave >> 2, k = wave & 3;
    const float *x = (const float *)xbuf;
    float sc = x[(b * 4 + k) * 64 + lane];
#pragma unroll
    for (int pp = 1; pp < R::kParts; ++pp) sc += x[((b + 2 * pp) * 4 + k) * 64 + lane];
    const bool valid = ((vmask >> (b * 16 + kbase + 2 * k)) & 1u) != 0;
    return valid ? __builtin_fmaf(sc, p.scale_log2, -m_run) : -INFINITY;
  };
  auto softmax_publish = [&](uint32_t vmask) {
    const float d = value_logit(vmask);
    publish(d, d > kRescaleSlack);
  };
  // Reads the 512 words of a tile whose partial scores are still in xbuf;
  // if any overshoots, moves the reference max to the tile's max, rescales
  // and republishes (every wave reads the same words, so all take the branch).
  auto consume_words = [&](uint32_t vmask, bf16x8 &p_hi, bf16x8 &p_lo) {
    uint32_t w[8];
    uint32_t flags = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      w[j] = *pword(j, lane);
      flags |= w[j];
    }
    if (__ballot((flags >> 31) != 0) != 0) {
      __builtin_amdgcn_s_barrier();  // all flags read before any word is rewritten
      f32x4 sacc[2];
      reduce(sacc);
      const float c = p.scale_log2;
      const uint32_t vm = vmask >> kbase;
      float mx = -INFINITY;
#pragma unroll
      for (int bb = 0; bb < 2; ++bb)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
          if ((vm >> (bb * 16 + 2 * kk)) & 1u) mx = fmaxf(mx, sacc[bb][kk] * c);
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run, mx);
      const float alpha = (m_run == -INFINITY) ? 0.f : fast_exp2(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int fb = 0; fb < R::kNFB; ++fb) acc[fb] *= alpha;
      publish(value_logit(vmask), false);
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
      __builtin_amdgcn_s_barrier();        // republished words visible, xbuf reads done
#pragma unroll
      for (int j = 0; j < 8; ++j) w[j] = *pword(j, lane);
    }
    l_run += pv_pending;  // this wave's share; the shares are added at the end
    // no word carries a flag here (none was set, or all were republished)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      p_hi[j] = __builtin_bit_cast(__bf16, (uint16_t)(w[j] >> 16));
      p_lo[j] = __builtin_bit_cast(__bf16, (uint16_t)(w[j] & 0xffffu));
    }
  };
  // O^T += V^T . P^T over this wave's feature slice, V from the tile at st_ckv
  auto pv = [&](const char *st_ckv, const bf16x8 &p_hi, const bf16x8 &p_lo) {
    // ---- O^T += V^T . P^T over this wave's feature slice; k-slot k of lane
    // group g is key kbase+2k (k < 4) or 16+kbase+2(k-4).  Lane 16g+s points
    // the transpose read at key row kbase + 2*(s/4) (+16 for slots 4..7),
    // features f0 + 4*(s%4).  Scheduling barriers every four feature blocks
    // keep the compiler from hoisting all reads of a wide slice (FS == 1:
    // 64 of them) ahead of the MFMAs.
    const char *vsrc = st_ckv + (kbase + 2 * (r16 >> 2)) * kCkvPitch +
                       (fs * R::kNFB * 16 + 4 * (r16 & 3)) * 2;
    // The reads are tr_read4 batches (inline asm): with the builtin form the
    // compiler waits for every outstanding LDS DMA (vmcnt(0)) before the
    // first read, which drains the gathers in flight on every tile.
    for_tr_batches<R::kNFB, 16 * kCkvPitch>(vsrc, [&](int f0, const bf16x8(&av)[4]) {
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[f], p_hi, acc[f0 + f], 0, 0, 0);
        acc[f0 + f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[f], p_lo, c, 0, 0, 0);
      }
    });
  };

  const int pre = min(n_tiles, kStages - 1);
  for (int j = 0; j < pre; ++j) fire_tile(j, tile_src(j));

  // the first ring pass's tile masks, built while the first tiles are in flight
  for (int k = 0; 2 * k < min(n_tiles, L::kRingTiles); ++k) {
    const int i = k * 64 + lane;
    const uint64_t bits = __ballot(i < n_tiles * kKeysPerTile && slots[i] >= 0);
    tile_masks = lane == 2 * k ? (uint32_t)bits : tile_masks;
    tile_masks = lane == 2 * k + 1 ? (uint32_t)(bits >> 32) : tile_masks;
  }

  // Waits until tile i has landed for this wave; the tiles issued after it
  // (up to kStages - 2 of them) may stay in flight.
  auto wait_tile = [&](int i) {
    static_assert(kStages == 4, "the waits below assume two tiles ahead");
    if (i + 2 < n_tiles)
      wait_vmcnt<2 * R::kLoads>();
    else if (i + 1 < n_tiles)
      wait_vmcnt<R::kLoads>();
    else
      wait_vmcnt<0>();
  };

  // Software pipeline: iteration i computes S^T of tile i and the PV
  // product of tile i-1, so the PV MFMAs overlap the latency chain of the
  // scores (LDS reads -> MFMA -> exchange).  The second barrier (the partial
  // exchange when FS > 1) also proves every wave done with tile i-1, whose
  // stage then receives tile i+3.  Tile i-1 stays in LDS one iteration
  // longer, which is what the fourth stage is for; two tiles remain in
  // flight.
  bf16x8 p_hi = {}, p_lo = {};
  int next_refill = 16;  // the next tile index whose issue triggers a slot-id refill
  for (int i = 0; i < n_tiles; ++i) {
    wait_tile(i);
    if constexpr (kShared) __builtin_amdgcn_s_waitcnt(0xC07F);  // this wave's words of tile i-1 written
    __builtin_amdgcn_s_barrier();  // every wave's share of tile i landed (and tile i-1's words)
    if constexpr (kShared)
      if (i > 0) consume_words(__builtin_amdgcn_readlane(tile_masks, i - 1), p_hi, p_lo);
    // stage offsets: tile i, and tile i-1 (whose stage receives tile i+3)
    const int st_cur = (i & (kStages - 1)) * kStageBytes;
    const int st_prev = ((i + kStages - 1) & (kStages - 1)) * kStageBytes;
    const char *st_ckv = lds + st_cur;
    f32x4 sacc[2];
    scores(st_ckv, sacc);
    if (i > 0) pv(lds + st_prev, p_hi, p_lo);
    if (FS >= 2) xput(sacc[0]);
    // (The one-slice layouts compute the addresses after the barrier: their
    // waves have no registers to hold them across it.)
    const bool refill_stage = i + kStages - 1 < n_tiles;
    TileSrc nxt;
    if (FS >= 2 && refill_stage) nxt = tile_src(i + kStages - 1);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): partial written, tile i-1 read
    __builtin_amdgcn_s_barrier();
    if (FS == 1 && refill_stage) nxt = tile_src(i + kStages - 1);
    if (refill_stage) fire_tile(i + kStages - 1, nxt);
    // Ring refill (layouts whose ring holds 32 tiles' ids): once tile J = 16 m
    // (m >= 1) is issued, every wave has passed a barrier since it read the
    // ids of tiles J - 16 .. J - 1, so their half of the ring takes the ids of
    // tiles J + 16 .. J + 31 (one 4-byte DMA per lane; raw ids, checked when
    // issued).  The DMA completes before the loads of tile J + 1 (in-order
    // vmcnt) and is visible after that tile's barrier, 14 iterations before
    // tile J + 16 is issued.  The stage waits meanwhile count one extra load,
    // which only makes them wait longer.
    if constexpr (FS >= 2) {
      static_assert(W == 8, "a half refill is 512 ids, one per lane of 8 waves");
      const int J = i + kStages - 1;
      if (J == next_refill) {  // J = 16, 32, ... (kept in a scalar, not tested per tile)
        next_refill += 16;
        if (J + 16 < n_tiles) {
          const int key = (J + 16) * kKeysPerTile + wave * 64 + lane;  // W == 8: 512 keys
          const int32_t *src = key < n_keys ? p.idx + (int64_t)t * p.idx_st + k_begin + key
                                            : g_minus_one + lane;
          lds_dma4(src, slots + ((J + 16) % L::kRingTiles) * kKeysPerTile + wave * 64);
        }
      }
    }
    if constexpr (kShared) {
      softmax_publish(__builtin_amdgcn_readlane(tile_masks, i));
    } else {
      if (FS >= 2) reduce(sacc);
      softmax(sacc, __builtin_amdgcn_readlane(tile_masks, i), p_hi, p_lo);
    }
  }
  if (n_tiles > 0) {
    if constexpr (kShared) {
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_s_barrier();  // the last tile's words visible
      consume_words(__builtin_amdgcn_readlane(tile_masks, n_tiles - 1), p_hi, p_lo);
    }
    pv(lds + ((n_tiles - 1) & (kStages - 1)) * kStageBytes, p_hi, p_lo);
  }

  // ---- epilogue: lanes of a head hold partial sums over disjoint keys (and,
  // with the probability exchange, each wave over its share of the values)
  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);
  if constexpr (kShared) {
    __builtin_amdgcn_s_barrier();  // every wave done with the exchange words
    if (lane < 16) *pword(wave >> 1, (wave & 1) * 32 + lane) = __float_as_uint(l_run);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    float l = 0.f;
#pragma unroll
    for (int w = 0; w < 8; ++w) l += __uint_as_float(*pword(w >> 1, (w & 1) * 32 + r16));
    l_run = l;
  }
  if (p.num_splits == 1 && !p.partial_only) {
    const float inv = (m_run == -INFINITY) ? 0.f : 1.f / l_run;
#pragma unroll
    for (int fb = 0; fb < R::kNFB; ++fb) {
      const int f0 = (fs * R::kNFB + fb) * 16 + 4 * g;
      bf16x4 ob;
#pragma unroll
      for (int k = 0; k < 4; ++k) ob[k] = (__bf16)(acc[fb][k] * inv);
      *(bf16x4 *)(p.out + t * p.out_st + head * p.out_sh + f0 * 2) = ob;
    }
    if (fs == 0 && lane < 16)
      p.lse[t * p.lse_st + head * p.lse_sh] =
          (m_run == -INFINITY) ? -INFINITY : m_run + __log2f(l_run);
    return;
  }

  // ---- split: write this chunk's partial
  const int S = p.num_splits;
  const int64_t prow = ((int64_t)t * S + split) * p.H + head;
  // (The in-kernel merge is built for the 8-slice layout only: with fewer
  // slices a wave owns more feature blocks, its merge takes one memory round
  // trip per 4 of them, and the tail costs more than the merge kernel.)
  if (FS != 8 || p.counters == nullptr) {  // dsa_attn_combine_kernel merges
#pragma unroll
    for (int fb = 0; fb < R::kNFB; ++fb) {
      const int f0 = (fs * R::kNFB + fb) * 16 + 4 * g;
      *(f32x4 *)(p.part_acc + prow * kHeadDimCkv + f0) = acc[fb];
    }
    if (fs == 0 && lane < 16) {
      p.part_ml[prow * 2 + 0] = m_run;
      p.part_ml[prow * 2 + 1] = l_run;
    }
    return;
  }

  if constexpr (FS == 8) {
  // ---- in-kernel merge.  A wave's feature slice of its head group depends
  // only on the same slice of the other chunks, so each wave counts arrivals
  // on its own counter (no workgroup-wide flag, no barrier) and exchanges its
  // partial through a private region in lane order (kNFB x 1 KB of acc, then
  // 16 (m, l) pairs), one contiguous 1 KB per store instruction.  The chunks
  // of a token run on different XCDs, whose L2s are not coherent with each
  // other.  A device-scope release/acquire fence pair would write back /
  // invalidate the whole L2 (buffer_wbl2 / buffer_inv), which costs more than
  // the second launch it saves; instead the exchange uses sc1 accesses
  // (device-coherent: written through to, and read from, the memory side, as
  // device-scope atomics are) and the wave waits for its stores to complete
  // (vmcnt(0); stores count there) before it draws a ticket.  The wave that
  // draws the last ticket resets the counter for the next launch and merges
  // the slice in split order with the merge kernel's arithmetic, so both
  // paths give the same bits whichever chunk finishes last.
  // Regions of workgroup (t, s, blockIdx.y): its W waves' acc regions tile
  // exactly the workgroup's share of part_acc (kHG x 16 heads x 512 fp32),
  // and its W x 16 (m, l) pairs fit in the share of part_ml the host sizes
  // (kHG x 16 heads x 8 pairs).
  static_assert(W * R::kNFB * 256 == R::kHG * kHeadsPerGroup * kHeadDimCkv, "acc regions");
  static_assert(W * 32 <= R::kHG * kHeadsPerGroup * 16, "(m, l) regions");
  const int64_t wg0 = (int64_t)t * S * gridDim.y + blockIdx.y;  // chunk s: + s * gridDim.y
  auto acc_region = [&](int s) {
    const int64_t w = ((wg0 + (int64_t)s * gridDim.y) * W + wave) * (R::kNFB * 256);
    return __builtin_amdgcn_make_buffer_rsrc(p.part_acc + w, 0, R::kNFB * 1024, kBufferFlags);
  };
  auto ml_region = [&](int s) {
    const int64_t w = ((wg0 + (int64_t)s * gridDim.y) * W + wave) * 32;
    return __builtin_amdgcn_make_buffer_rsrc(p.part_ml + w, 0, 128, kBufferFlags);
  };
  {
    const auto ar = acc_region(split);
#pragma unroll
    for (int fb = 0; fb < R::kNFB; ++fb)
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[fb]), ar,
                                             (fb * 64 + lane) * 16, 0, kSC1);
    if (lane < 16)
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, make_float2(m_run, l_run)),
                                            ml_region(split), lane * 8, 0, kSC1);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  uint32_t *cnt = p.counters + ((int64_t)t * gridDim.y + blockIdx.y) * 8 + wave;
  uint32_t ticket = 0;
  if (lane == 0) ticket = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  ticket = __shfl(ticket, 0);
  if (ticket != (uint32_t)(S - 1)) return;
  if (lane == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  auto load_ml = [&](int s) {
    return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(ml_region(s), r16 * 8, 0, kSC1));
  };
  constexpr int kB = 4;                           // chunks whose loads are in flight together
  constexpr int kF = R::kNFB < 4 ? R::kNFB : 4;   // feature blocks per load batch
  // The max over chunks comes first; with at most kB chunks it is taken from
  // the first load batch itself (one memory round trip fewer).
  float M = -INFINITY;
  for (int s0 = 0; S > kB && s0 < S; s0 += kB) {
    float mv[kB];
#pragma unroll
    for (int j = 0; j < kB; ++j) mv[j] = load_ml(min(s0 + j, S - 1)).x;
#pragma unroll
    for (int j = 0; j < kB; ++j) M = fmaxf(M, mv[j]);  // clamped repeats leave the max alone
  }
  // Feature blocks in batches of kF (bounded registers in the 1-slice
  // layouts); the sum L is complete after the first batch.
  float L = 0.f, inv = 0.f;
#pragma unroll
  for (int fc = 0; fc < R::kNFB; fc += kF) {
    f32x4 o[kF];
#pragma unroll
    for (int f = 0; f < kF; ++f) o[f] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < S; s0 += kB) {
      float a[kB];
      float2 ml[kB];
      f32x4 pa[kB][kF];
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        const int s = min(s0 + j, S - 1);
        ml[j] = load_ml(s);
        const auto ar = acc_region(s);
#pragma unroll
        for (int f = 0; f < kF; ++f)
          pa[j][f] = __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(ar, ((fc + f) * 64 + lane) * 16, 0, kSC1));
      }
      if (S <= kB) {
#pragma unroll
        for (int j = 0; j < kB; ++j) M = fmaxf(M, ml[j].x);
      }
#pragma unroll
      for (int j = 0; j < kB; ++j) {
        a[j] = (ml[j].x == -INFINITY) ? 0.f : fast_exp2(ml[j].x - M);
        if (fc == 0 && s0 + j < S) L += a[j] * ml[j].y;
      }
#pragma unroll
      for (int j = 0; j < kB; ++j)
        if (s0 + j < S) {
#pragma unroll
          for (int f = 0; f < kF; ++f) o[f] += a[j] * pa[j][f];
        }
    }
    if (fc == 0) inv = (M == -INFINITY) ? 0.f : 1.f / L;
#pragma unroll
    for (int f = 0; f < kF; ++f) {
      const int f0 = (fs * R::kNFB + fc + f) * 16 + 4 * g;
      bf16x4 ob;
#pragma unroll
      for (int k = 0; k < 4; ++k) ob[k] = (__bf16)(o[f][k] * inv);
      *(bf16x4 *)(p.out + t * p.out_st + head * p.out_sh + f0 * 2) = ob;
    }
  }
  if (fs == 0 && lane < 16)
    p.lse[t * p.lse_st + head * p.lse_sh] = (M == -INFINITY) ? -INFINITY : M + __log2f(L);
  }
}

// Log-sum-exp merge of the per-chunk partials (reference: dsa_reduce_kernel,
// kernel.py:437-493, with its -inf guards :475-476).  One workgroup per
// (token, head); 128 threads x 4 features.  Split order is fixed, so the
// result is deterministic.
// SMAX > 0: at most SMAX splits, all partial loads issued before any use (one
// memory round trip); SMAX == 0: any number of splits, loaded as consumed.
template <int SMAX>
__global__ __launch_bounds__(128) void dsa_attn_combine_kernel(AttnParams p) {
  const int t = blockIdx.x;
  const int head = blockIdx.y;
  const int S = p.num_splits;
  const int f0 = threadIdx.x * 4;
  const int64_t row0 = (int64_t)t * S * p.H + head;
  float M = -INFINITY, L = 0.f;
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
  if constexpr (SMAX > 0) {
    float2 ml[SMAX];
    f32x4 pa[SMAX];
#pragma unroll
    for (int s = 0; s < SMAX; ++s) {
      if (s < S) {
        const int64_t row = row0 + (int64_t)s * p.H;
        ml[s] = *(const float2 *)(p.part_ml + row * 2);
        pa[s] = *(const f32x4 *)(p.part_acc + row * kHeadDimCkv + f0);
      }
    }
#pragma unroll
    for (int s = 0; s < SMAX; ++s)
      if (s < S) M = fmaxf(M, ml[s].x);
#pragma unroll
    for (int s = 0; s < SMAX; ++s) {
      if (s < S) {
        const float a = (ml[s].x == -INFINITY) ? 0.f : fast_exp2(ml[s].x - M);
        L += a * ml[s].y;
        o += a * pa[s];
      }
    }
  } else {
    for (int s = 0; s < S; ++s) M = fmaxf(M, p.part_ml[(row0 + (int64_t)s * p.H) * 2]);
    for (int s = 0; s < S; ++s) {
      const int64_t row = row0 + (int64_t)s * p.H;
      const float ms = p.part_ml[row * 2];
      const float a = (ms == -INFINITY) ? 0.f : fast_exp2(ms - M);
      L += a * p.part_ml[row * 2 + 1];
      o += a * *(const f32x4 *)(p.part_acc + row * kHeadDimCkv + f0);
    }
  }
  const float inv = (M == -INFINITY) ? 0.f : 1.f / L;
  bf16x4 ob;
#pragma unroll
  for (int i = 0; i < 4; ++i) ob[i] = (__bf16)(o[i] * inv);
  *(bf16x4 *)(p.out + t * p.out_st + head * p.out_sh + f0 * 2) = ob;
  if (threadIdx.x == 0)
    p.lse[t * p.lse_st + head * p.lse_sh] = (M == -INFINITY) ? -INFINITY : M + __log2f(L);
}

template <int W, int FS>
hipError_t launch_ring(const AttnParams &p, int head_blocks, hipStream_t stream) {
  const dim3 grid(p.T * p.num_splits, head_blocks), block(W * 64);
  if (p.narrow)
    hipLaunchKernelGGL((dsa_attn_ring_kernel<W, FS, true>), grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL((dsa_attn_ring_kernel<W, FS, false>), grid, block, 0, stream, p);
  return hipGetLastError();
}

}  // namespace

bool attn_merges_in_kernel(int H) { return (H / kHeadsPerGroup) % 2 != 0; }  // the <8, 8> layout

int attn_max_chunk(int) {
  static_assert(Lds<1>::kMaxChunkKeys == Lds<8>::kMaxChunkKeys, "one chunk bound for every layout");
  return Lds<1>::kMaxChunkKeys;
}

int attn_head_blocks(int H) {
  const int groups = H / kHeadsPerGroup;
  if (groups % 8 == 0) return groups / 8;
  if (groups % 4 == 0) return groups / 4;
  if (groups % 2 == 0) return groups / 2;
  return groups;
}

hipError_t launch_attention_partial(const AttnParams &p, hipStream_t stream) {
  if (p.T == 0) return hipSuccess;
  const int groups = p.H / kHeadsPerGroup;
  const int hb = attn_head_blocks(p.H);
  if (groups % 8 == 0) return launch_ring<8, 1>(p, hb, stream);  // one wave per head group
  if (groups % 4 == 0) return launch_ring<4, 1>(p, hb, stream);
  if (groups % 2 == 0) return launch_ring<8, 4>(p, hb, stream);  // 2 groups x 4 slices
  return launch_ring<8, 8>(p, hb, stream);                       // 1 group x 8 slices
}

hipError_t launch_attention_merge(const AttnParams &p, hipStream_t stream) {
  if (p.T == 0) return hipSuccess;
  const dim3 grid(p.T, p.H), block(128);
  if (p.num_splits <= 4) hipLaunchKernelGGL(dsa_attn_combine_kernel<4>, grid, block, 0, stream, p);
  else if (p.num_splits <= 8) hipLaunchKernelGGL(dsa_attn_combine_kernel<8>, grid, block, 0, stream, p);
  else if (p.num_splits <= 16) hipLaunchKernelGGL(dsa_attn_combine_kernel<16>, grid, block, 0, stream, p);
  else hipLaunchKernelGGL(dsa_attn_combine_kernel<0>, grid, block, 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_attention(const AttnParams &pin, hipStream_t stream) {
  AttnParams p = pin;
  if (!attn_merges_in_kernel(p.H)) p.counters = nullptr;
  hipError_t e = launch_attention_partial(p, stream);
  if (e != hipSuccess || (p.num_splits == 1 && !p.partial_only) || p.counters != nullptr) return e;
  return launch_attention_merge(p, stream);
}

}  // namespace dsa
