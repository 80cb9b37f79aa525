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
// Two layouts, both one workgroup per (token, top-k chunk, block of head
// groups), both gathering the selected rows by LDS DMA (16 B per lane
// straight into LDS, no VGPR staging) with padding keys gathering a zero row,
// which keeps the number of loads per block fixed and makes the vmcnt-based
// stage waits exact.  Dense caches below 2 GB (every BASELINE shape) are
// gathered with buffer_load ... lds at 32-bit offsets slot * row stride (one
// 24-bit multiply per key, one readlane per row); a padding key's offset lies
// past the buffer's range, and an out-of-range buffer load returns zeros,
// which the DMA writes as the row.  Other caches take global_load_lds_dwordx4
// at 64-bit addresses, the page division as a multiply by a host-computed
// reciprocal, and a zero row in global memory.
//
// dsa_attn_wave_kernel (an odd number of 16-head groups: H = 16 decode and
// prefill; described at the kernel): four independent waves, each with a
// private two-stage ring of 16-key blocks and its keys in ascending slot
// order, merged through LDS at the end.
//
// dsa_attn_ring_kernel (H a multiple of 32): the waves share a 4-stage LDS
// ring of 32-key tiles (the whole 160 KB of LDS), two tiles in flight while
// two are in use.  The chunk's slot ids are staged in LDS (4 bytes per key,
// so no index load sits in front of a gather) and the valid-key mask of every
// tile is kept in one VGPR (lane i: tile i).  Each wave belongs to one
// 16-head group and owns one slice of the 512 output features.  Per tile:
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
// guards :475-476), so results are deterministic: in the wave layout inside
// the kernel by the wave that finishes a feature slice last (device-coherent
// sc1 stores and loads plus a per-wave arrival counter, no L2 write-back),
// otherwise by dsa_attn_combine_kernel.  Both give the same bits.
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
// kbase = 0, 8, 1, 9.  The QK operand reads touch 16 distinct rows and the PV
// transpose reads of one 32-lane half 8 rows whose 32-byte pieces land on
// disjoint bank ranges; the row layouts below keep both free of bank
// conflicts.
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

// LDS geometry (bytes).  gfx950's LDS serves a ds_read_b128 32 lanes at a
// time over 128 four-byte banks (512 bytes): the 32 lanes' 16-byte pieces must
// fall on distinct 16-byte columns of a 512-byte line (measured: a colliding
// pair doubles the instruction's LDS cycles).  An MFMA operand read takes
// 16-byte piece g of 16 rows in lane group g (g = 0, 1 in a half), so rows at a
// pitch of 1024 + 16 B put piece 1 of row r on the column of piece 0 of row
// r + 1.  The ring kernel keeps that pitch and stores key k of a 32-key tile
// at row ring_row(k) = 2 (k mod 16) + k / 16 (a 16-key block on every other
// row: columns 2r + g); the wave kernel holds 16-key blocks and pads its rows
// to 1024 + 32 B instead (kWavePitch).  Both place the transposing V^T reads
// (8-byte pieces, 32 lanes a time) on distinct columns as well.  kpe rows are
// gathered 8 per DMA instruction in chunk-major order (lane i of the DMA holds
// 16-byte chunk i/8 of row i%8); group q of a tile starts at
// kpe_group_off(q), odd groups 128 B further, so the two groups one 16-key
// block reads fall on different halves of the line.
constexpr int kCkvPitch = 1024 + 16;
constexpr int kKpeGroupPitch = 1024 + 128;
__device__ __forceinline__ int ring_row(int k) { return 2 * (k & 15) + (k >> 4); }
__device__ __forceinline__ int kpe_group_off(int q) { return q * kKpeGroupPitch + (q & 1) * 128; }
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

// Eight transposing reads (feature blocks F0 .. F0+7, 32 bytes apart) into
// o, left in flight: the caller's next tr_issue8_wait / tr_wait_all waits for
// them.  No LDS access may be issued between (the waits count LDS operations).
template <int F0>
__device__ __forceinline__ void tr_issue8(uint32_t va, u32x2 (&o)[8]) {
  asm volatile(
      "ds_read_b64_tr_b16 %0, %8 offset:%9\n\t"
      "ds_read_b64_tr_b16 %1, %8 offset:%10\n\t"
      "ds_read_b64_tr_b16 %2, %8 offset:%11\n\t"
      "ds_read_b64_tr_b16 %3, %8 offset:%12\n\t"
      "ds_read_b64_tr_b16 %4, %8 offset:%13\n\t"
      "ds_read_b64_tr_b16 %5, %8 offset:%14\n\t"
      "ds_read_b64_tr_b16 %6, %8 offset:%15\n\t"
      "ds_read_b64_tr_b16 %7, %8 offset:%16"
      : "=&v"(o[0]), "=&v"(o[1]), "=&v"(o[2]), "=&v"(o[3]), "=&v"(o[4]), "=&v"(o[5]), "=&v"(o[6]),
        "=&v"(o[7])
      : "v"(va), "i"(F0 * 32), "i"(F0 * 32 + 32), "i"(F0 * 32 + 64), "i"(F0 * 32 + 96),
        "i"(F0 * 32 + 128), "i"(F0 * 32 + 160), "i"(F0 * 32 + 192), "i"(F0 * 32 + 224)
      : "memory");
}

// tr_issue8<F0> into o, then waits until the previous batch `prev` (issued
// before it) has landed: its registers are in/out operands of the wait, so
// their uses cannot move above it.
template <int F0>
__device__ __forceinline__ void tr_issue8_wait(uint32_t va, u32x2 (&o)[8], u32x2 (&prev)[8]) {
  asm volatile(
      "ds_read_b64_tr_b16 %0, %16 offset:%17\n\t"
      "ds_read_b64_tr_b16 %1, %16 offset:%18\n\t"
      "ds_read_b64_tr_b16 %2, %16 offset:%19\n\t"
      "ds_read_b64_tr_b16 %3, %16 offset:%20\n\t"
      "ds_read_b64_tr_b16 %4, %16 offset:%21\n\t"
      "ds_read_b64_tr_b16 %5, %16 offset:%22\n\t"
      "ds_read_b64_tr_b16 %6, %16 offset:%23\n\t"
      "ds_read_b64_tr_b16 %7, %16 offset:%24\n\t"
      "s_waitcnt lgkmcnt(8)"
      : "=&v"(o[0]), "=&v"(o[1]), "=&v"(o[2]), "=&v"(o[3]), "=&v"(o[4]), "=&v"(o[5]), "=&v"(o[6]),
        "=&v"(o[7]), "+v"(prev[0]), "+v"(prev[1]), "+v"(prev[2]), "+v"(prev[3]), "+v"(prev[4]),
        "+v"(prev[5]), "+v"(prev[6]), "+v"(prev[7])
      : "v"(va), "i"(F0 * 32), "i"(F0 * 32 + 32), "i"(F0 * 32 + 64), "i"(F0 * 32 + 96),
        "i"(F0 * 32 + 128), "i"(F0 * 32 + 160), "i"(F0 * 32 + 192), "i"(F0 * 32 + 224)
      : "memory");
}

__device__ __forceinline__ void tr_wait_all(u32x2 (&prev)[8]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(prev[0]), "+v"(prev[1]), "+v"(prev[2]), "+v"(prev[3]), "+v"(prev[4]),
                 "+v"(prev[5]), "+v"(prev[6]), "+v"(prev[7])
               :
               : "memory");
}

// Q^T of one head group from its LDS staging (see the wave kernel): k-steps
// 0..15 at qn + 64 k, k-steps 16, 17 at qp and qp + 64, with the wait, in one
// asm statement (the compiler would wait for every LDS DMA in flight before
// the builtin form).
__device__ __forceinline__ void q_read18(uint32_t qn, uint32_t qp, bf16x8 (&q)[18]) {
  asm volatile(
      "ds_read_b128 %0, %18\n\t"
      "ds_read_b128 %1, %18 offset:64\n\t"
      "ds_read_b128 %2, %18 offset:128\n\t"
      "ds_read_b128 %3, %18 offset:192\n\t"
      "ds_read_b128 %4, %18 offset:256\n\t"
      "ds_read_b128 %5, %18 offset:320\n\t"
      "ds_read_b128 %6, %18 offset:384\n\t"
      "ds_read_b128 %7, %18 offset:448\n\t"
      "ds_read_b128 %8, %18 offset:512\n\t"
      "ds_read_b128 %9, %18 offset:576\n\t"
      "ds_read_b128 %10, %18 offset:640\n\t"
      "ds_read_b128 %11, %18 offset:704\n\t"
      "ds_read_b128 %12, %18 offset:768\n\t"
      "ds_read_b128 %13, %18 offset:832\n\t"
      "ds_read_b128 %14, %18 offset:896\n\t"
      "ds_read_b128 %15, %18 offset:960\n\t"
      "ds_read_b128 %16, %19\n\t"
      "ds_read_b128 %17, %19 offset:64\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(q[0]), "=&v"(q[1]), "=&v"(q[2]), "=&v"(q[3]), "=&v"(q[4]), "=&v"(q[5]), "=&v"(q[6]),
        "=&v"(q[7]), "=&v"(q[8]), "=&v"(q[9]), "=&v"(q[10]), "=&v"(q[11]), "=&v"(q[12]),
        "=&v"(q[13]), "=&v"(q[14]), "=&v"(q[15]), "=&v"(q[16]), "=&v"(q[17])
      : "v"(qn), "v"(qp)
      : "memory");
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

// Workgroup barrier for LDS data only: this wave's LDS accesses complete
// (lgkmcnt(0)), then s_barrier, in one statement the compiler moves no memory
// access across.  Unlike __syncthreads() it leaves vector-memory loads (and
// LDS DMAs) in flight.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ uint64_t readlane64(uint64_t v, int lane) {
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, lane);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), lane);
  return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// o += a * x with one rounding per component, written out: the split merges
// must give the same bits in every kernel, and an add that the compiler
// moves past a branch is no longer contracted with its product.
__device__ __forceinline__ void fma_to(f32x4 &o, float a, const f32x4 &x) {
#pragma unroll
  for (int k = 0; k < 4; ++k) o[k] = __builtin_fmaf(a, x[k], o[k]);
}

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

// Fused QK/PV loop (one-slice layouts, one head group per wave): S^T of
// both 16-key blocks of tile i interleaved with the PV product of tile i-1.
// Step K (0..35) is QK k-step K % 18 of key block K / 18 and, for K < 32,
// feature block K of the PV product (its V^T halves of key block 0 and 1).
// The reads of step K+1 are issued before the MFMAs of step K, so a step's
// LDS latency is covered by the previous step's MFMAs (1 QK + 2 PV), and
// consecutive MFMAs of one chain are never back to back.  qa*/ka*: LDS
// addresses of this lane's QK operand rows (ckv; kpe + 128 g) of key blocks
// 0 and 1; va: the V^T read address (as in the pv stage).
struct FusedAddr {
  uint32_t qa0, qa1, ka0, ka1, va;
};

template <int K>
__device__ __forceinline__ void fused_issue(const FusedAddr &a, u32x4 &kq, u32x2 (&vt)[2]) {
  constexpr int kRowB = kCkvPitch;  // key block 1 of the V^T reads: the next row (ring_row)
  constexpr int kStep = K % 18;
  constexpr int kOff = kStep < 16 ? kStep * 64 : (kStep - 16) * 512;
  const uint32_t qa = K < 18 ? (kStep < 16 ? a.qa0 : a.ka0) : (kStep < 16 ? a.qa1 : a.ka1);
  if constexpr (K < 32) {
    asm volatile(
        "ds_read_b128 %0, %3 offset:%4\n\t"
        "ds_read_b64_tr_b16 %1, %5 offset:%6\n\t"
        "ds_read_b64_tr_b16 %2, %5 offset:%7"
        : "=&v"(kq), "=&v"(vt[0]), "=&v"(vt[1])
        : "v"(qa), "i"(kOff), "v"(a.va), "i"(K * 32), "i"(kRowB + K * 32)
        : "memory");
  } else {
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=&v"(kq) : "v"(qa), "i"(kOff) : "memory");
  }
}

// Waits until at most N LDS operations issued after step K's reads are
// outstanding (LDS operations complete in issue order; any other operation
// counted meanwhile only makes the wait longer).  Step K's registers are
// in/out operands, so their uses cannot move above the wait.
template <int N, int K>
__device__ __forceinline__ void fused_wait(u32x4 &kq, u32x2 (&vt)[2]) {
  if constexpr (K < 32)
    asm volatile("s_waitcnt lgkmcnt(%3)" : "+v"(kq), "+v"(vt[0]), "+v"(vt[1]) : "n"(N) : "memory");
  else
    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(kq) : "n"(N) : "memory");
}

template <int K = 0>
__device__ __forceinline__ void qk_pv_steps(const FusedAddr &a, const QkOperands<1> &q, const bf16x8 &p_hi,
                                            const bf16x8 &p_lo, f32x4 (&acc)[32], f32x4 (&s)[2],
                                            u32x4 (&kq)[2], u32x2 (&vt)[2][2]) {
  if constexpr (K < 36) {
    constexpr int kNext = K + 1;
    if constexpr (kNext < 36) fused_issue<kNext>(a, kq[kNext & 1], vt[kNext & 1]);
    constexpr int kAfter = kNext < 36 ? (kNext < 32 ? 3 : 1) : 0;
    fused_wait<kAfter, K>(kq[K & 1], vt[K & 1]);
    constexpr int kStep = K % 18;
    const bf16x8 b = kStep < 16 ? q.nope[kStep] : q.pe32[kStep - 16];
    const bf16x8 ak = __builtin_bit_cast(bf16x8, kq[K & 1]);
    if constexpr (K < 32) {
      const bf16x8 av = __builtin_bit_cast(bf16x8, u32x4{vt[K & 1][0][0], vt[K & 1][0][1], vt[K & 1][1][0],
                                                         vt[K & 1][1][1]});
      acc[K] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, p_hi, acc[K], 0, 0, 0);
      s[K / 18] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak, b, s[K / 18], 0, 0, 0);
      acc[K] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, p_lo, acc[K], 0, 0, 0);
    } else {
      s[K / 18] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ak, b, s[K / 18], 0, 0, 0);
    }
    qk_pv_steps<K + 1>(a, q, p_hi, p_lo, acc, s, kq, vt);
  }
}

__device__ __forceinline__ void qk_pv_tile(const FusedAddr &a, const QkOperands<1> &q, const bf16x8 &p_hi,
                                           const bf16x8 &p_lo, f32x4 (&acc)[32], f32x4 (&s)[2]) {
  u32x4 kq[2];
  u32x2 vt[2][2];
  s[0] = f32x4{0.f, 0.f, 0.f, 0.f};
  s[1] = f32x4{0.f, 0.f, 0.f, 0.f};
  fused_issue<0>(a, kq[0], vt[0]);
  qk_pv_steps(a, q, p_hi, p_lo, acc, s, kq, vt);
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
  static_assert(FS == 1 || FS == 2 || FS == 4, "feature slices");
};

// A chunk's partial result from one wave: NFB feature blocks starting at
// block fs * NFB of the 16 heads of `head`'s group, with the (m, l) pair of
// each head.  Without split counters the partial goes to the layout of
// dsa_attn_combine_kernel ([T][S][H][512] and [T][S][H][2]; ml_writer: the
// one wave per head group that writes the pairs).  With counters the token's
// chunks are merged here: a wave's feature slice depends only on the same
// slice of the other chunks, so each wave counts arrivals on its own counter
// and exchanges its partial through a private region in lane order (NFB x
// 1 KB of acc, then 16 (m, l) pairs), one contiguous 1 KB per store
// instruction.  The chunks of a token run on different XCDs, whose L2s are
// not coherent with each other: the exchange uses sc1 accesses (device
// coherent: written through to, and read from, the memory side, as
// device-scope atomics are) and the wave waits for its stores to complete
// (vmcnt(0); stores count there) before it draws a ticket.  The wave that
// draws the last ticket resets the counter for the next launch and merges the
// slice in split order with the merge kernel's arithmetic, so both paths give
// the same bits whichever chunk finishes last.  Regions of workgroup (t, s,
// blockIdx.y): its W waves' acc regions tile exactly its share of part_acc
// (16 heads x 512 fp32 per head group) and its W x 16 pairs fit in the share
// of part_ml the host sizes (16 pairs per head).
template <int W, int NFB>
__device__ __forceinline__ void split_partial(const AttnParams &p, int t, int split, int head, int wave,
                                              int lane, int fs, const f32x4 (&acc)[NFB], float m_run,
                                              float l_run, bool ml_writer) {
  const int g = lane >> 4, r16 = lane & 15;
  const int S = p.num_splits;
  const int64_t prow = ((int64_t)t * S + split) * p.H + head;
  if (p.counters == nullptr) {
#pragma unroll
    for (int fb = 0; fb < NFB; ++fb) {
      const int f0 = (fs * NFB + fb) * 16 + 4 * g;
      *(f32x4 *)(p.part_acc + prow * kHeadDimCkv + f0) = acc[fb];
    }
    if (ml_writer && lane < 16) {
      p.part_ml[prow * 2 + 0] = m_run;
      p.part_ml[prow * 2 + 1] = l_run;
    }
    return;
  }
  static_assert(W * NFB * 256 == kHeadsPerGroup * kHeadDimCkv, "acc regions of one head group");
  static_assert(W * 32 <= kHeadsPerGroup * 16, "(m, l) regions");
  const int64_t wg0 = (int64_t)t * S * gridDim.y + blockIdx.y;  // chunk s: + s * gridDim.y
  auto acc_region = [&](int s) {
    const int64_t w = ((wg0 + (int64_t)s * gridDim.y) * W + wave) * (NFB * 256);
    return __builtin_amdgcn_make_buffer_rsrc(p.part_acc + w, 0, NFB * 1024, kBufferFlags);
  };
  auto ml_region = [&](int s) {
    const int64_t w = ((wg0 + (int64_t)s * gridDim.y) * W + wave) * 32;
    return __builtin_amdgcn_make_buffer_rsrc(p.part_ml + w, 0, 128, kBufferFlags);
  };
  {
    const auto ar = acc_region(split);
#pragma unroll
    for (int fb = 0; fb < NFB; ++fb)
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
  // lane 0's ticket as a scalar: kept in a VGPR, the compiler substitutes it
  // for S - 1 below and the buffer resources built from it become per-lane
  // values, each load then wrapped in a waterfall loop
  ticket = __builtin_amdgcn_readfirstlane(ticket);
  if (ticket != (uint32_t)(S - 1)) return;
  if (lane == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  auto load_ml = [&](int s) {
    return __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(ml_region(s), r16 * 8, 0, kSC1));
  };
  constexpr int kB = 4;    // chunks whose loads are in flight together
  constexpr int kF = NFB;  // feature blocks per load batch: all of the wave's
  // The max over chunks comes first (16 chunks' pairs per round trip); with
  // at most kB chunks it is taken from the first load batch itself (one
  // memory round trip fewer).
  float M = -INFINITY;
  for (int s0 = 0; S > kB && s0 < S; s0 += 16) {
    float mv[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) mv[j] = load_ml(min(s0 + j, S - 1)).x;
#pragma unroll
    for (int j = 0; j < 16; ++j) M = fmaxf(M, mv[j]);  // clamped repeats leave the max alone
  }
  // Feature blocks in batches of kF; the sum L is complete after the first.
  float L = 0.f, inv = 0.f;
#pragma unroll
  for (int fc = 0; fc < NFB; fc += kF) {
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
        if (fc == 0 && s0 + j < S) L = __builtin_fmaf(a[j], ml[j].y, L);
      }
#pragma unroll
      for (int j = 0; j < kB; ++j)
        if (s0 + j < S) {
#pragma unroll
          for (int f = 0; f < kF; ++f) fma_to(o[f], a[j], pa[j][f]);
        }
    }
    if (fc == 0) inv = (M == -INFINITY) ? 0.f : 1.f / L;
#pragma unroll
    for (int f = 0; f < kF; ++f) {
      const int f0 = (fs * NFB + fc + f) * 16 + 4 * g;
      bf16x4 ob;
#pragma unroll
      for (int k = 0; k < 4; ++k) ob[k] = (__bf16)(o[f][k] * inv);
      *(bf16x4 *)(p.out + t * p.out_st + head * p.out_sh + f0 * 2) = ob;
    }
  }
  if (ml_writer && lane < 16)
    p.lse[t * p.lse_st + head * p.lse_sh] = (M == -INFINITY) ? -INFINITY : M + __log2f(L);
}

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

  // The fused QK/PV loop of the one-slice layouts runs a PV step on the
  // first tile too, from the stage of tile -1 with zero probabilities: that
  // stage's ckv rows are zeroed here (its first gather is issued after the
  // first tile is computed), so the step adds exact zeros.
  if constexpr (FS == 1) {
    u32x4 *z = (u32x4 *)(lds + (kStages - 1) * kStageBytes);
    for (int i = threadIdx.x; i < kCkvStageBytes / 16; i += W * 64) z[i] = u32x4{0u, 0u, 0u, 0u};
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
    char *kdst = st + kCkvStageBytes + kpe_group_off(grp);
    if constexpr (NARROW) {
#pragma unroll
      for (int m = 0; m < R::kRows; ++m)
        lds_dma16_buf(ckv_rsrc, st + ring_row(grp * 8 + row0 + m) * kCkvPitch, a.row[m] + lane * 16);
      if (kpe_lane) lds_dma16_buf(kpe_rsrc, kdst, a.ko);
    } else {
#pragma unroll
      for (int m = 0; m < R::kRows; ++m) {
        const char *src = (const char *)readlane64(a.ckv, row0 + m) + lane * 16;
        lds_dma16(src, st + ring_row(grp * 8 + row0 + m) * kCkvPitch);
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
      const char *rowp = st_ckv + ring_row(kk) * kCkvPitch + g * 16;
      const char *kp = st_kpe + kpe_group_off(kk >> 3) + (kk & 7) * 16;
      sacc[bb] = qk_part<R::kParts>(part, rowp, kp, qreg, g);
    }
  };
  // Partial S^T exchange: slot w holds wave w's partial of its key block.
  auto xput = [&](const f32x4 &v) { xbuf[wave * 64 + lane] = v; };
  auto xget = [&](int slot) -> f32x4 { return xbuf[slot * 64 + lane]; };
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
  // O^T += V^T . P^T over this wave's feature slice, V from the tile at st_ckv
  auto pv = [&](const char *st_ckv, const bf16x8 &p_hi, const bf16x8 &p_lo) {
    // ---- O^T += V^T . P^T over this wave's feature slice; k-slot k of lane
    // group g is key kbase+2k (k < 4) or 16+kbase+2(k-4).  Lane 16g+s points
    // the transpose read at key kbase + 2*(s/4) (+16 for slots 4..7: the next
    // LDS row, ring_row), features f0 + 4*(s%4).  Scheduling barriers every four feature blocks
    // keep the compiler from hoisting all reads of a wide slice (FS == 1:
    // 64 of them) ahead of the MFMAs.
    const char *vsrc = st_ckv + ring_row(kbase + 2 * (r16 >> 2)) * kCkvPitch +
                       (fs * R::kNFB * 16 + 4 * (r16 & 3)) * 2;
    // The reads are tr_read4 batches (inline asm): with the builtin form the
    // compiler waits for every outstanding LDS DMA (vmcnt(0)) before the
    // first read, which drains the gathers in flight on every tile.
    for_tr_batches<R::kNFB, kCkvPitch>(vsrc, [&](int f0, const bf16x8(&av)[4]) {
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[f], p_hi, acc[f0 + f], 0, 0, 0);
        acc[f0 + f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av[f], p_lo, c, 0, 0, 0);
      }
    });
  };

  // two teams of waves (W == 8, one-slice): waves 0-3 and 4-7, one of each
  // per SIMD, half an iteration apart (below); they keep two tiles ahead
  constexpr bool kTeams = FS == 1 && W == 8;
  const int pre = min(n_tiles, kTeams ? 2 : kStages - 1);
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
  auto lds_addr = [](const char *q) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char *)q;
  };
  const int k0 = key_of_row(r16), k1 = 16 + key_of_row(r16);
  if constexpr (kTeams) {
    const bool team_b = wave >= 4;
    f32x4 sb[2];  // S^T of the wave's current tile, from its QK/PV step to its softmax
    auto fused = [&](int i, f32x4 (&sacc)[2]) {
      const char *st_ckv = lds + (i & (kStages - 1)) * kStageBytes;
      const char *st_prev = lds + ((i + kStages - 1) & (kStages - 1)) * kStageBytes;
      const char *st_kpe = st_ckv + kCkvStageBytes;
      const FusedAddr fa = {
          lds_addr(st_ckv + ring_row(k0) * kCkvPitch + g * 16), lds_addr(st_ckv + ring_row(k1) * kCkvPitch + g * 16),
          lds_addr(st_kpe + kpe_group_off(k0 >> 3) + (k0 & 7) * 16 + g * 128),
          lds_addr(st_kpe + kpe_group_off(k1 >> 3) + (k1 & 7) * 16 + g * 128),
          lds_addr(st_prev + ring_row(kbase + 2 * (r16 >> 2)) * kCkvPitch + 4 * (r16 & 3) * 2)};
      qk_pv_tile(fa, qreg, p_hi, p_lo, acc, sacc);
    };
    // Both teams run the same loop (X_j, fused j, Y_j, softmax j); team B
    // passes one extra barrier first and team A one after, so the barriers
    // pair A's X_j with B's Y_{j-1} and A's Y_j with B's X_j: each team's
    // QK/PV of a tile runs while the other team does its softmax.  Before a
    // barrier that lets either team compute tile j, both teams' shares of
    // tile j have landed: A waits before X_j, B before Y_{j-1}.  The stage of
    // tile j-2 is free once both teams passed their fused step j-1, i.e.
    // after the pair (A's X_j, B's Y_{j-1}): B fires its share of tile j+2
    // right after that pair (before its softmax of tile j-1), A after its
    // softmax of tile j (while B runs its fused step j).
    int fired = pre - 1;  // last tile whose share this wave has issued
    auto wait_own = [&](int j) {  // this wave's share of tile j landed
      const int ahead = fired - j;
      if (ahead >= 2)
        wait_vmcnt<2 * R::kLoads>();
      else if (ahead == 1)
        wait_vmcnt<R::kLoads>();
      else
        wait_vmcnt<0>();
    };
    if (team_b) {
      // this barrier is team A's X_0: team B's share of tile 0 lands first
      wait_own(0);
      __builtin_amdgcn_s_barrier();
      if (2 < n_tiles) {
        fire_tile(2, tile_src(2));
        fired = 2;
      }
    }
    for (int j = 0; j < n_tiles; ++j) {
      wait_own(j);
      __builtin_amdgcn_s_barrier();  // X_j
      fused(j, sb);
      if (team_b && j + 1 < n_tiles) wait_own(j + 1);
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_s_barrier();  // Y_j
      if (team_b && j + 3 < n_tiles) {
        fire_tile(j + 3, tile_src(j + 3));
        fired = j + 3;
      }
      softmax(sb, __builtin_amdgcn_readlane(tile_masks, j), p_hi, p_lo);
      // team A issues its share of tile j+2 here, where it waits for team B's
      // QK/PV anyway, not between X_j and its own QK/PV
      if (!team_b && j + 2 < n_tiles) {
        fire_tile(j + 2, tile_src(j + 2));
        fired = j + 2;
      }
    }
    if (!team_b) __builtin_amdgcn_s_barrier();
  } else {
    int next_refill = 16;  // the next tile index whose issue triggers a slot-id refill
    for (int i = 0; i < n_tiles; ++i) {
      wait_tile(i);
      __builtin_amdgcn_s_barrier();  // every wave's share of tile i landed
      // stage offsets: tile i, and tile i-1 (whose stage receives tile i+3)
      const int st_cur = (i & (kStages - 1)) * kStageBytes;
      const int st_prev = ((i + kStages - 1) & (kStages - 1)) * kStageBytes;
      const char *st_ckv = lds + st_cur;
      f32x4 sacc[2];
      if constexpr (FS == 1) {
        // S^T of tile i fused with the PV product of tile i-1 (tile 0: the PV
        // part reads the zeroed stage with zero probabilities)
        const char *st_kpe = st_ckv + kCkvStageBytes;
        const FusedAddr fa = {
            lds_addr(st_ckv + ring_row(k0) * kCkvPitch + g * 16), lds_addr(st_ckv + ring_row(k1) * kCkvPitch + g * 16),
            lds_addr(st_kpe + kpe_group_off(k0 >> 3) + (k0 & 7) * 16 + g * 128),
            lds_addr(st_kpe + kpe_group_off(k1 >> 3) + (k1 & 7) * 16 + g * 128),
            lds_addr(lds + st_prev + ring_row(kbase + 2 * (r16 >> 2)) * kCkvPitch + 4 * (r16 & 3) * 2)};
        qk_pv_tile(fa, qreg, p_hi, p_lo, acc, sacc);
      } else {
        scores(st_ckv, sacc);
        if (i > 0) pv(lds + st_prev, p_hi, p_lo);
      }
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
      if (FS >= 2) reduce(sacc);
      softmax(sacc, __builtin_amdgcn_readlane(tile_masks, i), p_hi, p_lo);
    }
  }
  if (n_tiles > 0) pv(lds + ((n_tiles - 1) & (kStages - 1)) * kStageBytes, p_hi, p_lo);

  // ---- epilogue: lanes of a head hold partial sums over disjoint keys
  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);
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

  // ---- split: this chunk's partial for dsa_attn_combine_kernel (these
  // layouts never merge inside the kernel: a wave owns 8 or more feature
  // blocks, so an in-kernel merge costs more memory round trips than the
  // second launch)
  const int64_t prow = ((int64_t)t * p.num_splits + split) * p.H + head;
#pragma unroll
  for (int fb = 0; fb < R::kNFB; ++fb) {
    const int f0 = (fs * R::kNFB + fb) * 16 + 4 * g;
    *(f32x4 *)(p.part_acc + prow * kHeadDimCkv + f0) = acc[fb];
  }
  if (fs == 0 && lane < 16) {
    p.part_ml[prow * 2 + 0] = m_run;
    p.part_ml[prow * 2 + 1] = l_run;
  }
}

// ---- one head group: four independent waves --------------------------------
//
// Layout for head counts of an odd number of 16-head groups (H = 16 decode
// and prefill): one workgroup per (token, top-k chunk, head group) with four
// waves, one per SIMD.  Each wave owns a quarter of the chunk's 16-key blocks
// (from 16 blocks on its keys taken in ascending slot order) and runs on its
// own: its blocks are gathered by LDS DMA into a private two-stage ring
// (block j+1 in flight while block j is computed), its scores
// are complete (the whole 576-wide QK per wave: no partial-score exchange),
// and its online softmax and O^T accumulator cover its own keys only.  No
// workgroup barrier sits in the loop, so a wave waiting for a slow gather
// does not hold the others.  After the loop the four partial results are
// merged through LDS with log-sum-exp weights in wave order.
//
// Per block (16 keys):
//   S^T[16 keys x 16 heads] = K[keys x 576] . Q^T   18 x MFMA 16x16x32 bf16
//   O^T[512 x 16 heads]    += V^T[512 x keys] . P^T 32 x MFMA 16x16x32 bf16
// (P in bf16 hi + lo parts, both in one product: k-slots 8g..8g+3 hi,
// 8g+4..8g+7 lo).  MFMA row m of S^T is key key_of_row(m); the D layout of
// S^T (lane 16g + c: rows 4g..4g+3 of head c) gives lane group g the P^T
// values of key rows 4g..4g+3, whose V^T values (the A operand, repeated for
// the lo slots) are one ds_read_b64_tr_b16 per feature block.
//
// Stage layout: 16 ckv rows at a 1056-byte pitch (key k at row k), then the
// 16 kpe rows chunk-major (16-byte chunk c of key k at 256 c + 16 k), so the
// QK operand reads (16 rows, one column) and the transposing V^T reads (rows
// key_of_row(4g + j)) are free of bank conflicts.
constexpr int kWavePitch = 1024 + 32;
constexpr int kWaveBlock = 16;                          // keys per block
constexpr int kWaveWaves = 4;
constexpr int kWaveKpeOff = kWaveBlock * kWavePitch;     // 16896
constexpr int kWaveStage = kWaveKpeOff + kWaveBlock * 128;  // + 2048 = 18944
constexpr int kWaveRing = 2 * kWaveStage;
constexpr int kWaveIds = kMaxChunkWide;                 // slot ids of a chunk, staged once
constexpr int kWaveSortBlocks = 16;  // a wave sorts its keys by slot from this many blocks on
constexpr int kWaveLds = kWaveWaves * kWaveRing + kWaveIds * 4;
static_assert(kWaveLds <= 160 * 1024, "LDS budget of one gfx950 CU");
// the merge after the loop reuses each wave's ring: three 8 KB slices (one
// per other wave), then 16 (m, l) pairs
static_assert(3 * 8192 + 16 * 8 <= kWaveRing, "merge space");

template <bool NARROW>
__global__ __launch_bounds__(kWaveWaves * 64, 1) void dsa_attn_wave_kernel(AttnParams p) {
  __shared__ __attribute__((aligned(16))) char lds[kWaveLds];
  int32_t *slots = (int32_t *)(lds + kWaveWaves * kWaveRing);

  const int t = blockIdx.x / p.num_splits;
  const int split = blockIdx.x - t * p.num_splits;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int head = blockIdx.y * kHeadsPerGroup + r16;
  const int k_begin = split * p.chunk;
  const int n_keys = max(0, min(p.K, k_begin + p.chunk) - k_begin);
  const int n_blocks = (n_keys + kWaveBlock - 1) / kWaveBlock;
  const int b0 = n_blocks * wave / kWaveWaves;  // this wave's blocks: [b0, b1)
  const int my_blocks = n_blocks * (wave + 1) / kWaveWaves - b0;
  char *ring = lds + wave * kWaveRing;

  // Prologue: this wave's ids are loaded (and, on long runs, sorted), its
  // quarter of the workgroup's Q is staged in LDS, the first gather is
  // issued, and Q^T is read into registers from the staging.
  constexpr int kPer = kWaveIds / (kWaveWaves * 64);  // ids per lane (a wave takes <= 512 keys)
  const int32_t *isrc = p.idx + (int64_t)t * p.idx_st + k_begin + b0 * kWaveBlock;
  const int n_mine = my_blocks * kWaveBlock;  // keys of this wave's blocks (tail padding included)
  const int n_real = min(n_mine, n_keys - b0 * kWaveBlock);
  int sv[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int i = k * 64 + lane;
    sv[k] = i < n_real ? isrc[i] : -1;
  }
  auto valid_id = [&](int s) { return (s >= 0 && (int64_t)s < p.num_slots) ? s : -1; };

  int32_t *my_ids = slots + wave * (kWaveIds / kWaveWaves);
  if (my_blocks < kWaveSortBlocks) {
    // few blocks: the keys keep their given order (the sort below costs
    // about 1 us of the prologue and pays only on long runs)
#pragma unroll
    for (int k = 0; k < kPer; ++k)
      if (k * 64 + lane < n_mine) my_ids[k * 64 + lane] = valid_id(sv[k]);
  } else {
    // ---- order this wave's keys by slot: a stable counting sort on the top 8
    // bits of the slot id (256 buckets, each a contiguous range of the cache),
    // in the wave's own (not yet used) ring, so no workgroup barrier is
    // needed: one wave's LDS accesses execute in program order.  Every wave of
    // every workgroup then sweeps the cache upwards at the same time, which
    // keeps address translation and cache lines shared between neighbouring
    // gathers.  The order depends on the ids alone: results stay
    // deterministic.  Scratch: per-vector bucket counts hist[k][256] (bytes;
    // vector k = keys 64k .. 64k+63 of the wave), their start positions
    // start[k][256] (u16); the sorted ids go to the wave's 512-entry slice of
    // the id array.
    uint8_t *hist = (uint8_t *)ring;
    uint16_t *start = (uint16_t *)(ring + kPer * 256);
    static_assert(kPer * 256 * 3 <= kWaveRing, "sort scratch in the ring");
    *(u32x4 *)(hist + lane * 32) = u32x4{0u, 0u, 0u, 0u};
    *(u32x4 *)(hist + lane * 32 + 16) = u32x4{0u, 0u, 0u, 0u};
    const uint32_t top = (uint32_t)min(p.num_slots, (int64_t)0x7fffffff);
    const int shift = max(0, (32 - __builtin_clz(max(top, 1u))) - 8);
    int bk[kPer], rk[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int id = valid_id(sv[k]);
      sv[k] = id;
      const int b = k * 64 + lane < n_mine ? (id >= 0 ? (id >> shift) : 255) : -1;
      bk[k] = b;
      rk[k] = 0;
      if (k * 64 < n_mine) {  // wave-uniform
        uint64_t same = __ballot(b >= 0);
#pragma unroll
        for (int bit = 0; bit < 8; ++bit) {
          const bool on = (b >> bit) & 1;
          const uint64_t bb = __ballot(on);
          same &= on ? bb : ~bb;
        }
        const int rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(same >> 32),
                                                   __builtin_amdgcn_mbcnt_lo((uint32_t)same, 0));
        rk[k] = rank;
        if (b >= 0 && rank == __popcll(same) - 1) hist[k * 256 + b] = (uint8_t)(rank + 1);
      }
    }
    {
      // lane l owns buckets 4l .. 4l+3
      uint32_t pre[kPer][4], tot[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int k = 0; k < kPer; ++k) {
        const uint32_t c4 = *(const uint32_t *)(hist + k * 256 + lane * 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          pre[k][i] = tot[i];
          tot[i] += (c4 >> (8 * i)) & 255u;
        }
      }
      const int lsum = (int)(tot[0] + tot[1] + tot[2] + tot[3]);
      int incl = lsum;
      incl += __builtin_amdgcn_update_dpp(0, incl, 0x111, 0xf, 0xf, false);  // row_shr:1
      incl += __builtin_amdgcn_update_dpp(0, incl, 0x112, 0xf, 0xf, false);  // row_shr:2
      incl += __builtin_amdgcn_update_dpp(0, incl, 0x114, 0xf, 0xf, false);  // row_shr:4
      incl += __builtin_amdgcn_update_dpp(0, incl, 0x118, 0xf, 0xf, false);  // row_shr:8
      incl += __builtin_amdgcn_update_dpp(0, incl, 0x142, 0xa, 0xf, false);  // row_bcast:15
      incl += __builtin_amdgcn_update_dpp(0, incl, 0x143, 0xc, 0xf, false);  // row_bcast:31
      uint32_t base[4];
      base[0] = (uint32_t)(incl - lsum);
#pragma unroll
      for (int i = 1; i < 4; ++i) base[i] = base[i - 1] + tot[i - 1];
#pragma unroll
      for (int k = 0; k < kPer; ++k) {
        const uint32_t lo = (base[0] + pre[k][0]) | ((base[1] + pre[k][1]) << 16);
        const uint32_t hi = (base[2] + pre[k][2]) | ((base[3] + pre[k][3]) << 16);
        *(u32x2 *)(start + k * 256 + lane * 4) = u32x2{lo, hi};
      }
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k)
      if (bk[k] >= 0) my_ids[start[k * 256 + bk[k]] + rk[k]] = sv[k];
  }
  // ---- Q of the head group, staged once per workgroup (a quarter of the
  // traffic of every wave loading all of it, and issued after the ids are
  // stored, so the id loads that store waits for are not queued behind it;
  // issued right after the id loads instead it gained nothing): wave w DMAs the
  // q_nope rows of heads 4w .. 4w+3 (at the stage's row pitch: the 16 heads'
  // reads of one k-step land on distinct banks) and their q_pe rows (pitch 128)
  // into the second stage of wave 0's ring, which the loop first fills with
  // wave 0's second block.
  char *qstage = lds + kWaveStage;
  constexpr int kQPePos = kHeadsPerGroup * kWavePitch;  // q_pe rows after the 16 q_nope rows
  static_assert(kQPePos + kHeadsPerGroup * 128 <= kWaveStage, "Q staging fits one stage");
  {
    const int hb = blockIdx.y * kHeadsPerGroup;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 4 * wave + i;
      lds_dma16(p.q_nope + t * p.qn_st + (hb + h) * p.qn_sh + lane * 16, qstage + h * kWavePitch);
    }
    if (lane < 32) {
      const int h = 4 * wave + (lane >> 3);
      lds_dma16(p.q_pe + t * p.qp_st + (hb + h) * p.qp_sh + (lane & 7) * 16,
                qstage + kQPePos + 4 * wave * 128);
    }
  }
  const int id0 = my_blocks > 0 ? my_ids[r16] : -1;

  const auto ckv_rsrc = __builtin_amdgcn_make_buffer_rsrc((void *)p.ckv, 0, (int)p.ckv_extent, kBufferFlags);
  const auto kpe_rsrc = __builtin_amdgcn_make_buffer_rsrc((void *)p.kpe, 0, (int)p.kpe_extent, kBufferFlags);
  constexpr uint32_t kOOB = 0x80000000u;

  // Gather of a block into stage st, `id` being the slot of key r16 of the
  // block (-1: padding): 16 ckv rows (one 1 KB DMA each, the row's offset
  // read from its lane) and the kpe rows in two DMAs (lane l: chunk l/16 (+4)
  // of key l%16).  Returns the block's valid-key mask (bit k: key k).  Every
  // block issues exactly 18 loads, so the stage waits below are exact vmcnt
  // counts.
  auto gather = [&](int id, int st) -> uint32_t {
    char *dst = ring + st * kWaveStage;
    const uint32_t valid = (uint32_t)__ballot(id >= 0) & 0xffffu;
    if constexpr (NARROW) {
      const uint32_t co = id >= 0 ? __umul24((uint32_t)id, p.ckv_rs) : kOOB;
      const uint32_t ko = (id >= 0 ? __umul24((uint32_t)id, p.kpe_rs) : kOOB) + g * 16;
#pragma unroll
      for (int m = 0; m < kWaveBlock; ++m)
        lds_dma16_buf(ckv_rsrc, dst + m * kWavePitch, __builtin_amdgcn_readlane(co, m) + lane * 16);
      lds_dma16_buf(kpe_rsrc, dst + kWaveKpeOff, ko);
      lds_dma16_buf(kpe_rsrc, dst + kWaveKpeOff + 1024, ko + 64);
    } else {
      uint64_t ca = (uint64_t)(const char *)g_zero_row, ka = (uint64_t)(const char *)g_zero_row;
      if (id >= 0) {
        const uint32_t pg = (uint32_t)(((uint64_t)(uint32_t)id * p.ps_magic) >> (31 + p.ps_shift));
        const uint32_t of = (uint32_t)id - pg * (uint32_t)p.page_size;
        ca = (uint64_t)(p.ckv + (int64_t)pg * p.ckv_sp + (int64_t)of * p.ckv_so);
        ka = (uint64_t)(p.kpe + (int64_t)pg * p.kpe_sp + (int64_t)of * p.kpe_so);
      }
      ka += g * 16;
#pragma unroll
      for (int m = 0; m < kWaveBlock; ++m)
        lds_dma16((const char *)readlane64(ca, m) + lane * 16, dst + m * kWavePitch);
      lds_dma16((const char *)ka, dst + kWaveKpeOff);
      lds_dma16((const char *)ka + 64, dst + kWaveKpeOff + 1024);
    }
    return valid;
  };
  uint32_t vm_next = my_blocks > 0 ? gather(id0, 0) : 0u;
  // Q^T, the B operand of S^T = K Q^T: k-step k < 16 holds q_nope features
  // 32k + 8g .. +7 of head `head`, k-steps 16, 17 the q_pe features.  Every
  // wave's staging DMAs (issued before its first gather) have landed after
  // its wait and the barrier; the second barrier frees the staging for wave
  // 0's second block.
  if (my_blocks > 0)
    wait_vmcnt<18>();
  else
    wait_vmcnt<0>();
  __builtin_amdgcn_s_barrier();
  bf16x8 q[18];
  q_read18((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char *)(qstage + r16 * kWavePitch + g * 16),
           (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char *)(qstage + kQPePos + r16 * 128 + g * 16),
           q);
  __builtin_amdgcn_s_barrier();

  f32x4 acc[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;  // reference max (log2 units) of this lane's head over this wave's keys
  float l_run = 0.f;        // this lane's share of the sum
  const float c_log2 = p.scale_log2;
  // MFMA rows 4g..4g+3 of S^T are keys key_of_row(4g + i)
  int kor[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) kor[i] = key_of_row(4 * g + i);
  // QK operand rows: MFMA row r16 is key key_of_row(r16)
  const int qrow = key_of_row(r16);
  // transposing V^T reads: lanes 4j..4j+3 of group g point at key
  // key_of_row(4g + j), 8-byte piece (lane & 3) of the feature block
  const int vrow = key_of_row(4 * g + (r16 >> 2));
  const int voff = vrow * kWavePitch + (r16 & 3) * 8;

  for (int j = 0; j < my_blocks; ++j) {
    const int st = j & 1;
    const uint32_t vmask = vm_next;
    // the next block goes to the other stage (its block j-1 was consumed in
    // the previous iteration: every LDS read of it has completed)
    if (j + 1 < my_blocks) {
      vm_next = gather(my_ids[(j + 1) * kWaveBlock + r16], st ^ 1);
      wait_vmcnt<18>();
    } else {
      wait_vmcnt<0>();
    }
    const char *stg = ring + st * kWaveStage;

    // ---- S^T of the block (two accumulation chains)
    // (all 18 operand reads are issued before the first MFMA, so they cost
    // one LDS round trip, not one each)
    f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
    {
      const char *rowp = stg + qrow * kWavePitch + g * 16;
      const char *kp = stg + kWaveKpeOff + qrow * 16 + g * 256;
      bf16x8 ka[18];
#pragma unroll
      for (int k = 0; k < 16; ++k) ka[k] = *(const bf16x8 *)(rowp + k * 64);
      ka[16] = *(const bf16x8 *)kp;
      ka[17] = *(const bf16x8 *)(kp + 1024);
#pragma unroll
      for (int k = 0; k < 18; k += 2) {
        s0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[k], q[k], s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[k + 1], q[k + 1], s1, 0, 0, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 18, 0);  // DS reads
      __builtin_amdgcn_sched_group_barrier(0x008, 18, 0);  // then the MFMAs
    }
    // the first batch of transposing V^T reads goes out now: its latency
    // overlaps the softmax
    const uint32_t va = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char *)(stg + voff);
    u32x2 b0[8], b1[8], b2[8], b3[8];
    tr_issue8<0>(va, b0);
    const f32x4 s = s0 + s1;

    // ---- online softmax (log2 domain, reference max moved lazily)
    float d[4];
    bool over = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool ok = (vmask >> kor[i]) & 1u;
      d[i] = ok ? __builtin_fmaf(s[i], c_log2, -m_run) : -INFINITY;
      over |= d[i] > kRescaleSlack;
    }
    if (__ballot(over) != 0) {  // wave-uniform, rare after the first block
      float mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if ((vmask >> kor[i]) & 1u) mx = fmaxf(mx, s[i] * c_log2);
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run, mx);
      const float alpha = (m_run == -INFINITY) ? 0.f : fast_exp2(m_run - m_new);
      m_run = m_new;
      l_run *= alpha;
#pragma unroll
      for (int fb = 0; fb < 32; ++fb) acc[fb] *= alpha;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool ok = (vmask >> kor[i]) & 1u;
        d[i] = ok ? __builtin_fmaf(s[i], c_log2, -m_run) : -INFINITY;
      }
    }
    bf16x4 p_hi, p_lo;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float pv = fast_exp2(d[i]);
      l_run += pv;
      p_hi[i] = (__bf16)pv;
      p_lo[i] = (__bf16)(pv - (float)p_hi[i]);
    }
    // P^T as one 16x16x32 B operand: k-slots 8g .. 8g+3 of lane group g
    // hold the hi parts of key rows 4g .. 4g+3, k-slots 8g+4 .. 8g+7 their lo
    // parts, so P = hi + lo costs one MFMA per feature block (a 16x16x16
    // product takes as many cycles as a 16x16x32 one).
    const bf16x8 pb = __builtin_shufflevector(p_hi, p_lo, 0, 1, 2, 3, 4, 5, 6, 7);

    // ---- O^T += V^T . P^T in four batches of eight feature blocks: the
    // transposing reads of batch b+1 are issued before batch b's MFMAs.  The
    // A operand repeats the four V^T values of key rows 4g .. 4g+3 for the
    // lo k-slots.
    auto pv8 = [&](int f0, const u32x2 (&v)[8]) {
#pragma unroll
      for (int f = 0; f < 8; ++f) {
        const bf16x8 a = __builtin_bit_cast(bf16x8, u32x4{v[f][0], v[f][1], v[f][0], v[f][1]});
        acc[f0 + f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb, acc[f0 + f], 0, 0, 0);
      }
    };
    tr_issue8_wait<8>(va, b1, b0);
    pv8(0, b0);
    tr_issue8_wait<16>(va, b2, b1);
    pv8(8, b1);
    tr_issue8_wait<24>(va, b3, b2);
    pv8(16, b2);
    tr_wait_all(b3);
    pv8(24, b3);
  }

  // ---- merge the four waves' partials through LDS.  A wave's ring is free
  // once its own loop is done, so each wave writes its (m, l) pairs and the
  // unscaled feature blocks the other waves own into its own ring, and one
  // barrier later every wave adds up its blocks in wave order.
  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);
  // in ring(src): the 8 KB slice for wave dst at slot (dst - (dst > src)),
  // lane order (1 KB per feature block), then 16 (m, l) pairs
  auto slice = [&](int src, int dst) -> f32x4 * {
    return (f32x4 *)(lds + src * kWaveRing + (dst - (dst > src)) * 8192);
  };
  auto pairs = [&](int src) -> float2 * { return (float2 *)(lds + src * kWaveRing + 3 * 8192); };
  if (lane < 16) pairs(wave)[lane] = make_float2(m_run, l_run);
#pragma unroll
  for (int dst = 0; dst < kWaveWaves; ++dst) {
    if (dst == wave) continue;
    f32x4 *sl = slice(wave, dst);
#pragma unroll
    for (int f = 0; f < 8; ++f) sl[f * 64 + lane] = acc[dst * 8 + f];
  }
  lds_barrier();
  // Every read is issued before the first use (one LDS round trip): the four
  // (m, l) pairs and the slices the other three waves wrote for this one.
  float2 pr[kWaveWaves];
#pragma unroll
  for (int w = 0; w < kWaveWaves; ++w) pr[w] = pairs(w)[r16];
  f32x4 oth[kWaveWaves - 1][8];
#pragma unroll
  for (int i = 0; i < kWaveWaves - 1; ++i) {
    const f32x4 *sl = slice(i + (i >= wave), wave);
#pragma unroll
    for (int f = 0; f < 8; ++f) oth[i][f] = sl[f * 64 + lane];
  }
  // M and L in wave order, so every wave of the workgroup gets the same bits
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kWaveWaves; ++w) M = fmaxf(M, pr[w].x);
  float L = 0.f, aw[kWaveWaves];
#pragma unroll
  for (int w = 0; w < kWaveWaves; ++w) {
    aw[w] = (pr[w].x == -INFINITY) ? 0.f : fast_exp2(pr[w].x - M);
    L += aw[w] * pr[w].y;
  }
  // this wave's own blocks first, then the other waves' in ascending order (a
  // fixed order for each wave: deterministic sums); static register indices,
  // one uniform branch per wave
  f32x4 o[8];
#pragma unroll
  for (int w = 0; w < kWaveWaves; ++w)
    if (w == wave) {
#pragma unroll
      for (int f = 0; f < 8; ++f) o[f] = aw[w] * acc[w * 8 + f];
    }
#pragma unroll
  for (int i = 0; i < kWaveWaves - 1; ++i) {
    const float a = i < wave ? aw[i] : aw[i + 1];
#pragma unroll
    for (int f = 0; f < 8; ++f) o[f] += a * oth[i][f];
  }

  if (p.num_splits == 1 && !p.partial_only) {
    const float inv = (M == -INFINITY) ? 0.f : 1.f / L;
#pragma unroll
    for (int f = 0; f < 8; ++f) {
      const int f0 = (wave * 8 + f) * 16 + 4 * g;
      bf16x4 ob;
#pragma unroll
      for (int k = 0; k < 4; ++k) ob[k] = (__bf16)(o[f][k] * inv);
      *(bf16x4 *)(p.out + t * p.out_st + head * p.out_sh + f0 * 2) = ob;
    }
    if (wave == 0 && lane < 16)
      p.lse[t * p.lse_st + head * p.lse_sh] = (M == -INFINITY) ? -INFINITY : M + __log2f(L);
    return;
  }
  split_partial<kWaveWaves, 8>(p, t, split, head, wave, lane, wave, o, M, L, wave == 0);
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
        L = __builtin_fmaf(a, ml[s].y, L);
        fma_to(o, a, pa[s]);
      }
    }
  } else {
    for (int s = 0; s < S; ++s) M = fmaxf(M, p.part_ml[(row0 + (int64_t)s * p.H) * 2]);
    for (int s = 0; s < S; ++s) {
      const int64_t row = row0 + (int64_t)s * p.H;
      const float ms = p.part_ml[row * 2];
      const float a = (ms == -INFINITY) ? 0.f : fast_exp2(ms - M);
      L = __builtin_fmaf(a, p.part_ml[row * 2 + 1], L);
      fma_to(o, a, *(const f32x4 *)(p.part_acc + row * kHeadDimCkv + f0));
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

hipError_t launch_wave(const AttnParams &p, int head_blocks, hipStream_t stream) {
  const dim3 grid(p.T * p.num_splits, head_blocks), block(kWaveWaves * 64);
  if (p.narrow)
    hipLaunchKernelGGL(dsa_attn_wave_kernel<true>, grid, block, 0, stream, p);
  else
    hipLaunchKernelGGL(dsa_attn_wave_kernel<false>, grid, block, 0, stream, p);
  return hipGetLastError();
}

}  // namespace

bool attn_merges_in_kernel(int H, int64_t S) {
  return (H / kHeadsPerGroup) % 2 != 0 && S <= kMaxInKernelMergeSplits;
}

bool attn_wave_layout(int64_t T, int H, int64_t S) {
  const int groups = H / kHeadsPerGroup;
  return groups % 2 != 0 || T * S * groups <= kNumCU;
}

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
  // Odd group counts, and even ones whose workgroups of one group fit the
  // CUs in one round (small-T decode: H=128, top-k 2048, T=1 21.5 -> 14.1
  // us, T=4 28.6 -> 19.2 us; H=64 T=8 24.9 -> 19.0 us): four independent
  // waves per head group and chunk, no gathers shared between head groups.
  if (attn_wave_layout(p.T, p.H, p.num_splits)) return launch_wave(p, groups, stream);
  if (groups % 8 == 0) {
    // Four-wave workgroups of four head groups each -- twice the workgroups
    // of the eight-wave layout, each gathering the chunk's keys -- finish
    // sooner while that grid fits the CUs in one round (H=128, top-k 2048:
    // T=16 with 8 splits 35.1 us against 41.7 us for eight-wave workgroups
    // and 16 splits, T=32 with 4 splits 49.6 against 53.0 us; the same
    // bits); past that the eight-wave workgroups' shared gathers win.
    if ((int64_t)p.T * p.num_splits * (groups / 4) <= kNumCU)
      return launch_ring<4, 1>(p, groups / 4, stream);
    return launch_ring<8, 1>(p, hb, stream);  // one wave per head group
  }
  if (groups % 4 == 0) return launch_ring<4, 1>(p, hb, stream);
  return launch_ring<8, 4>(p, hb, stream);  // 2 groups x 4 slices
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
  if (!attn_merges_in_kernel(p.H, p.num_splits)) p.counters = nullptr;
  hipError_t e = launch_attention_partial(p, stream);
  if (e != hipSuccess || (p.num_splits == 1 && !p.partial_only) || p.counters != nullptr) return e;
  return launch_attention_merge(p, stream);
}

}  // namespace dsa
