// dsa_indexer.hip -- lightning-indexer scores and per-row top-k for gfx950.
//
// Score (the structure of the reference's indexer_kernel,
// solution/triton/indexer_kernel.py:185-275: dequantise -> dot -> ReLU ->
// head weight -> sum over heads; BASELINE config 5 form):
//
//   score[t,s] = sum_h w[t,h] * relu(q[t,h,:] . k[s,:] * k_scale[s])
//
// computed in the factored form k_scale[s] * sum_h w[t,h] * relu(d[t,s,h])
// (equal for a positive quantisation scale) with one exact rounding order, so
// the GPU reproduces the CPU oracle bit for bit:
//   D_h = d * 2^18, the exact integer dot of the values times 2^9;
//   r_h = fl32(max(D_h, 0));
//   the heads form 4 groups of Hi/4 consecutive heads; group g sums
//   G_g = fma(w_h, r_h, G_g) over its heads in ascending order from 0;
//   total = fl32(fl32(G_0 + G_1) + fl32(G_2 + G_3));
//   score = fl32(total * c_s), c_s = fl32(k_scale[s] * 2^-18).
// Positions beyond causal_limit[t] score -inf and are never selected.
//
// Exact dot on int8 MFMA.  Every finite e4m3fn value times 2^9 is an integer
// x with |x| <= 229376 (18 bits); x = p0 + 2^7 p1 + 2^14 p2 with signed 7-bit
// pieces (sign-magnitude split), so
//   D = sum_{a,b} 2^(7(a+b)) sum_j pq_a[j] pk_b[j]
// where each inner 128-term sum (|.| <= 128*127*127) is exact in the int32
// accumulator of v_mfma_i32_16x16x64_i8.  When every |x| < 2^14 (values below
// 32) the third piece is zero and D = P00 + 2^7 X + 2^14 P11 (X the two cross
// products) is combined in int32 when the operand maxima bound |D| below
// 2^31, else in fp64.  Where a whole range of positions allows the int32
// combine, three products suffice: the pieces lie in [0, 127] with the
// value's sign, so q1 - q0 and k0 - k1 fit int8 and C3 = P00 + (q1 - q0).(k0
// - k1) = X - P11 gives D = ((C3 + 129 P11) << 7) + P00.  Larger values take
// nine products and an fp64 combine (exact: every partial sum stays below
// 2^50).  e4m3fn NaN codes (0x7f, 0xff) count as zero.
//
// Kernels:
//   dsa_idx_prep_kernel    k codes -> piece planes laid out as MFMA
//                          operands in lane order (one 1 KB chunk per 16
//                          positions, piece and 64-wide k-step), plus the
//                          largest |x| of every 16-position block, and c_s
//                          of every position (kept by the caller as prepared
//                          K planes, or in the call's workspace).  With a
//                          paged K cache it reads each position's codes and
//                          scale through the page map.
//   dsa_idx_score_kernel   two waves per query token, up to 4 tokens per
//                          workgroup sharing a range of positions.  The
//                          token's q pieces are derived from its codes in
//                          registers (A operands, heads as M, through a code
//                          -> pieces table in LDS); each 16-position block's k pieces are
//                          one coalesced 1 KB load per operand (B, positions
//                          as N).  When every block of the range takes the
//                          three-product int32 path, the token's two waves
//                          claim chunks of six blocks from a counter in LDS
//                          and the loop is software-pipelined: a head block's
//                          MFMAs are issued beside the epilogue of the head
//                          block two before it.
//   dsa_idx_topk_kernel    one workgroup per row, the row in registers
//                          (loaded coalesced, 1024-strided, through one
//                          buffer descriptor): two radix passes (8 bits each,
//                          histograms replicated 32 ways so equal digits do
//                          not collide in one LDS bank) find the 16-bit bin
//                          of the k-th largest order key; keys above it are
//                          taken and the bin's few survivors are ranked
//                          exactly (key, then lower position first), else
//                          two more passes pin the k-th key and its ties go
//                          lowest positions first (reference intent:
//                          indexer_kernel.py:289-343, strict '>' keeps the
//                          earlier index).  The selection is a position
//                          bitmap built from ballots; one scan turns it into
//                          ranks in ascending position order.
//   dsa_idx_topk_stream_kernel  the four-pass selection re-reading the row
//                          from memory, for rows longer than 32768 positions.
//   dsa_k_append_kernel    quantise-on-append into the paged fp8 K cache:
//                          one wave per token (per-token fp32 scale from the
//                          row's largest magnitude, e4m3 round to nearest
//                          even).
#include <algorithm>

#include "../../include/dsa_abi.h"
#include "dsa_internal.h"

namespace dsa {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kIdxDim = 128;
constexpr int kKTokenBytes = kIdxDim + 4;  // paged K cache: codes + fp32 scale per token
constexpr int kChunk = 1024;              // one MFMA operand: 64 lanes x 16 bytes
constexpr int kBlockBytes = 3 * 2 * kChunk;  // k block: 3 planes x 2 k-steps
constexpr int kPrepThreads = 256;         // four waves, one destination block each
constexpr int kScoreWaves = 8;            // waves per score workgroup (two per token)
constexpr int kTargetScoreWaves = 2048;   // two waves per SIMD on 256 CUs
constexpr int kMinBlocksPerWave = 8;
constexpr int kTopkThreads = 1024;
constexpr int kMaxRegEpt = 32;            // register top-k up to 1024 * 32 positions
constexpr int kHistCopies = 32;
constexpr int kHistPitch = 257;           // copy c of bin j at c*257 + j: bank (c + j) % 64
constexpr int kTwoPieceLimit = 1 << 14;
constexpr int kBufferFlags = 0x00020000;  // raw buffer descriptor: 32-bit data format

// e4m3fn code -> x = value * 2^9 (integer), NaN codes -> 0.
__device__ __forceinline__ int e4m3_x(uint32_t c) {
  const int e = (c >> 3) & 15, m = c & 7;
  int x = (e == 0) ? m : ((8 + m) << (e - 1));
  if (e == 15 && m == 7) x = 0;
  return (c & 0x80) ? -x : x;
}

// Signed 7-bit piece `pc` of x (sign-magnitude split), as a byte.  The
// pieces of one value share its sign, so for |x| < 2^14 the difference
// p0 - p1 of its two pieces lies in [-127, 127] as well.
__device__ __forceinline__ uint32_t piece_byte(int x, int pc) {
  const int mag = x < 0 ? -x : x;
  const int v = (mag >> (7 * pc)) & 127;
  return (uint32_t)(x < 0 ? -v : v) & 0xffu;
}

__device__ __forceinline__ i32x4 load_chunk(const int8_t *p) { return *(const i32x4 *)p; }

__device__ __forceinline__ i32x4 mfma(i32x4 a, i32x4 b, i32x4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// ---- operand preparation -------------------------------------------------

// e4m3fn code -> its signed 7-bit pieces as bytes: p0 | p1 << 8 | p2 << 16 |
// (p0 - p1) << 24 (the kernels keep this table in LDS).
__device__ __forceinline__ uint32_t piece_word(uint32_t code) {
  const int x = e4m3_x(code);
  const uint32_t b0 = piece_byte(x, 0), b1 = piece_byte(x, 1);
  const uint32_t d = (uint32_t)((int)(int8_t)b0 - (int)(int8_t)b1) & 0xffu;
  return b0 | (b1 << 8) | (piece_byte(x, 2) << 16) | (d << 24);
}

// Largest |x| (x = value * 2^9) of a set of codes from its largest code &
// 0x7f (e4m3 magnitudes order like their codes; the NaN code 0x7f ranks above
// 448, which only makes a bound conservative).
__device__ __forceinline__ int magnitude_bound(uint32_t top) {
  return top == 0x7f ? (15 << 14) : e4m3_x(top);
}

// Wave-wide largest code & 0x7f of the 32 codes a lane holds in w[8].
__device__ __forceinline__ uint32_t wave_top_code(const uint32_t (&w)[8]) {
  uint32_t mc = 0;
#pragma unroll
  for (int i = 0; i < 32; ++i) mc = max(mc, (w[i >> 2] >> (8 * (i & 3))) & 0x7fu);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mc = max(mc, (uint32_t)__shfl_xor((int)mc, o));
  return __builtin_amdgcn_readfirstlane(mc);
}

// Plane `byte` of the LUT words v[32] of a lane's 2 x 16 codes (negated: the
// plane's bytes negated), as the two k-steps' 16-byte operand pieces.
__device__ __forceinline__ void pack_plane(const uint32_t (&v)[32], int byte, bool negate,
                                           i32x4 (&out)[2]) {
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      uint32_t packed = 0;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        uint32_t x = (v[16 * ks + 4 * d + b] >> (8 * byte)) & 0xffu;
        if (negate) x = (0u - x) & 0xffu;
        packed |= x << (8 * b);
      }
      out[ks][d] = (int)packed;
    }
  }
}

// K blocks k_block0 .. k_block0 + k_blocks - 1 (16 positions each) -> piece
// planes laid out as MFMA B operands in lane order (one 1 KB chunk per plane
// and 64-wide k-step), the largest |x| of every block, and c_s of every
// position.  One wave per block; lane l = 16*g + c loads the 2 x 16 bytes it
// writes: position 16*block + c at dims 64*ks + 16*g for k-steps ks = 0, 1,
// so every plane store of the wave is one contiguous 1 KB chunk.  Positions
// at or past S read as zeros.
__global__ __launch_bounds__(kPrepThreads) void dsa_idx_prep_kernel(IndexerParams p) {
  __shared__ uint32_t lut[256];
  lut[threadIdx.x] = piece_word(threadIdx.x);
  __syncthreads();
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wblk = blockIdx.x * (kPrepThreads / 64) + wave;
  if (wblk >= p.k_blocks) return;
  const int blk = p.k_block0 + wblk;

  uint4 raw[2] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
  const int s = blk * 16 + c;
  if (s < p.S) {
    if (p.k_cache != nullptr) {  // paged: codes and scale through the page map
      const int pg = p.k_pages[s / p.k_page_size], off = s % p.k_page_size;
      if ((uint32_t)pg < (uint32_t)p.k_num_pages) {
        const uint8_t *page = p.k_cache + (int64_t)pg * p.k_page_size * kKTokenBytes;
        raw[0] = *(const uint4 *)(page + off * kIdxDim + g * 16);
        raw[1] = *(const uint4 *)(page + off * kIdxDim + 64 + g * 16);
        if (g == 0) p.k_cs[s] = *(const float *)(page + p.k_page_size * kIdxDim + off * 4) * 0x1p-18f;
      } else if (g == 0) {  // unmapped page: a zero row of scale 0
        p.k_cs[s] = 0.0f;
      }
    } else {
      const uint8_t *row = p.k + (int64_t)s * kIdxDim;
      raw[0] = *(const uint4 *)(row + g * 16);
      raw[1] = *(const uint4 *)(row + 64 + g * 16);
      if (g == 0) p.k_cs[s] = p.k_scale[s] * 0x1p-18f;
    }
  }
  int8_t *dst = p.k_pieces + (int64_t)blk * kBlockBytes + lane * 16;
  const uint32_t w[8] = {raw[0].x, raw[0].y, raw[0].z, raw[0].w, raw[1].x, raw[1].y, raw[1].z, raw[1].w};
  const int bmax = magnitude_bound(wave_top_code(w));
  if (lane == 0) p.k_max[blk] = bmax;

  uint32_t v[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) v[i] = lut[(w[i >> 2] >> (8 * (i & 3))) & 0xffu];
  // p0, p1, then p2 if the block holds a value of magnitude >= 32, else
  // p0 - p1 (slot 2 is read as p2 only for such blocks); non-temporal stores:
  // the planes are read by the next kernel, and stores kept in L2 cost a
  // write-back at the kernel's end (measured: 1.6 us of 10.8)
  const int bytes[3] = {0, 1, bmax < kTwoPieceLimit ? 3 : 2};
#pragma unroll
  for (int slot = 0; slot < 3; ++slot) {
    i32x4 o[2];
    pack_plane(v, bytes[slot], false, o);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      __builtin_nontemporal_store(__builtin_bit_cast(u32x4, o[ks]),
                                  (u32x4 *)(dst + (slot * 2 + ks) * kChunk));
  }
}

// The A operands of token t's head block hb, derived in registers from the
// raw codes: lane l = 16*g + c holds MFMA row c, which stands for head
// (c / 4) * Hi/4 + 4*hb + c % 4 (so the four output rows a lane receives,
// rows 4g..4g+3, are consecutive heads of head group g), dims 64*ks + 16*g ..
// +15 for k-steps ks = 0, 1.  Planes NPL of them, by LUT byte (4: p1 - p0).
template <int NPL>
__device__ __forceinline__ void q_operands(const IndexerParams &p, const uint32_t *lut, int t, int hb,
                                           const int (&plane)[NPL], i32x4 (&out)[NPL][2]) {
  const int lane = threadIdx.x & 63, c = lane & 15, g = lane >> 4;
  const int head = (c >> 2) * (p.Hi >> 2) + 4 * hb + (c & 3);
  const uint8_t *row = p.q + ((int64_t)t * p.Hi + head) * kIdxDim;
  const uint4 r0 = *(const uint4 *)(row + g * 16), r1 = *(const uint4 *)(row + 64 + g * 16);
  const uint32_t w[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
  uint32_t v[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) v[i] = lut[(w[i >> 2] >> (8 * (i & 3))) & 0xffu];
#pragma unroll
  for (int k = 0; k < NPL; ++k) pack_plane(v, plane[k] == 4 ? 3 : plane[k], plane[k] == 4, out[k]);
}

// Largest |x| over every code of token t (all heads), the same in every lane.
__device__ __forceinline__ int q_magnitude_bound(const IndexerParams &p, int t) {
  const int lane = threadIdx.x & 63;
  const uint4 *src = (const uint4 *)(p.q + (int64_t)t * p.Hi * kIdxDim);
  const int n16 = p.Hi * kIdxDim / 16;  // 16-byte pieces of the token's codes
  uint32_t mc = 0;
  for (int i = lane; i < n16; i += 64) {
    const uint4 r = src[i];
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int j = 0; j < 16; ++j) mc = max(mc, (w[j >> 2] >> (8 * (j & 3))) & 0x7fu);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mc = max(mc, (uint32_t)__shfl_xor((int)mc, o));
  return magnitude_bound(__builtin_amdgcn_readfirstlane(mc));
}

// ---- scores --------------------------------------------------------------

// (G0 + G1) + (G2 + G3) over the four 16-lane rows; every lane gets the sum.
// permlane16_swap exchanges rows 0<->1 and 2<->3, permlane32_swap the two
// halves; fp32 addition is commutative, so both lanes of a pair agree.
__device__ __forceinline__ float sum_lane_groups(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const float s = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Scores of token t over the 16-position blocks [b0, b1).  NQP = pieces of
// q in play (3 when the token holds a value of magnitude >= 32).
template <int NHB, int NQP>
__device__ __forceinline__ void score_range(const IndexerParams &p, const uint32_t *lut, int t, int b0,
                                            int b1, int qmax) {
  // The rounding order is part of the score's definition: no contraction of
  // the products and sums written below into fused multiply-adds (the one
  // fused step of the definition is the explicit fmaf).
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63;
  const int col = lane & 15, g = lane >> 4;
  const int lim = p.limit[t];
  float *srow = p.scores + (int64_t)t * p.S;
  uint32_t sh7;
  asm volatile("s_mov_b32 %0, 7" : "=s"(sh7));

  // A operands of this token: [head block][piece][k-step]
  i32x4 qa[NHB][NQP][2];
  {
    int planes[NQP];
#pragma unroll
    for (int pc = 0; pc < NQP; ++pc) planes[pc] = pc;
#pragma unroll
    for (int hb = 0; hb < NHB; ++hb) q_operands<NQP>(p, lut, t, hb, planes, qa[hb]);
  }
  // weights of the lane's rows: heads g*Hi/4 + 4*hb + i
  float wl[NHB][4];
  const float *wsrc = p.w + (int64_t)t * p.Hi + g * (p.Hi >> 2);
#pragma unroll
  for (int hb = 0; hb < NHB; ++hb)
#pragma unroll
    for (int i = 0; i < 4; ++i) wl[hb][i] = wsrc[4 * hb + i];

  // Blocks are fetched two ahead: pieces 0 and 1, the lane's scale, the
  // block's magnitude bound.  Indices past the range are clamped so every
  // step issues the same loads.
  struct KBlock {
    i32x4 k[2][2];
    float cs;
    int kmax;
  };
  auto fetch = [&](int b, KBlock &kb) {
    b = min(b, b1 - 1);
    const int8_t *src = p.k_pieces + (int64_t)b * kBlockBytes + lane * 16;
#pragma unroll
    for (int pc = 0; pc < 2; ++pc)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) kb.k[pc][ks] = load_chunk(src + (pc * 2 + ks) * kChunk);
    kb.cs = p.k_cs[min(b * 16 + col, p.S - 1)];
    kb.kmax = p.k_max[b];
  };

  // the lane's group sum for its position -> the score, stored by lanes 0..15
  auto finish = [&](float G, float cs, int s) {
    const float total = sum_lane_groups(G);
    const float score = total * cs;
    if (g == 0 && s >= 0 && s < p.S) srow[s] = (s > lim) ? -INFINITY : score;
  };
  // int32 combine of one head block's products into the lane's group sum:
  // D = ((P11 * 2^7 + X) * 2^7) + P00, two v_lshl_add_u32.  The shift amount
  // is an opaque scalar so that the compiler keeps this nesting instead of
  // redistributing the shifts into two shifts and an add3.
  auto epilogue = [&](const i32x4 &P00, const i32x4 &X, const i32x4 &P11, int hb, float &G) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t hi = ((uint32_t)P11[i] << sh7) + (uint32_t)X[i];
      const int D = (int)((hi << sh7) + (uint32_t)P00[i]);
      G = __builtin_fmaf(wl[hb][i], (float)max(D, 0), G);
    }
  };
  auto two_piece = [&](const i32x4 (&kc)[2][2], int hb, i32x4 &P00, i32x4 &X, i32x4 &P11) {
    const i32x4 z = {0, 0, 0, 0};
    P00 = mfma(qa[hb][0][1], kc[0][1], mfma(qa[hb][0][0], kc[0][0], z));
    X = mfma(qa[hb][0][0], kc[1][0], z);
    X = mfma(qa[hb][0][1], kc[1][1], X);
    X = mfma(qa[hb][1][0], kc[0][0], X);
    X = mfma(qa[hb][1][1], kc[0][1], X);
    P11 = mfma(qa[hb][1][1], kc[1][1], mfma(qa[hb][1][0], kc[1][0], z));
  };

  // fp64 combine (exact for every |D| < 2^53) of the general cases
  auto general = [&](const KBlock &kc, int b, int s, bool two) {
    float G = 0.f;
    if (NQP == 2 && two) {
#pragma unroll
      for (int hb = 0; hb < NHB; ++hb) {
        i32x4 P00, X, P11;
        two_piece(kc.k, hb, P00, X, P11);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const double D = (double)P00[i] + 128.0 * (double)X[i] + 16384.0 * (double)P11[i];
          G = __builtin_fmaf(wl[hb][i], (float)(D > 0.0 ? D : 0.0), G);
        }
      }
    } else {
      // all piece products, grouped by the power 2^(7(a+c)) they carry
      i32x4 kb3[3][2];
      const int8_t *src = p.k_pieces + (int64_t)b * kBlockBytes + lane * 16;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        kb3[0][ks] = kc.k[0][ks];
        kb3[1][ks] = kc.k[1][ks];
        kb3[2][ks] = kc.kmax >= kTwoPieceLimit ? load_chunk(src + (4 + ks) * kChunk)
                                               : i32x4{0, 0, 0, 0};
      }
#pragma unroll
      for (int hb = 0; hb < NHB; ++hb) {
        i32x4 C[5];
#pragma unroll
        for (int d = 0; d < 5; ++d) C[d] = i32x4{0, 0, 0, 0};
#pragma unroll
        for (int a = 0; a < NQP; ++a)
#pragma unroll
          for (int c = 0; c < 3; ++c)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) C[a + c] = mfma(qa[hb][a][ks], kb3[c][ks], C[a + c]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const double D = (double)C[0][i] + 0x1p7 * (double)C[1][i] + 0x1p14 * (double)C[2][i] +
                           0x1p21 * (double)C[3][i] + 0x1p28 * (double)C[4][i];
          G = __builtin_fmaf(wl[hb][i], (float)(D > 0.0 ? D : 0.0), G);
        }
      }
    }
    finish(G, kc.cs, s);
  };

  KBlock ka, kb, kc3;
  fetch(b0, ka);
  fetch(b0 + 1, kb);

  // One block: prefetch block b+2 into `ahead`, then score block b from `kc`.
  // Returns false once the rest of the range is causally masked.  The loop
  // below is unrolled by three so that the three buffers keep fixed roles
  // (a rotation by copies would wait for the loads just issued).
  auto step = [&](int b, const KBlock &kc, KBlock &ahead) -> bool {
    fetch(b + 2, ahead);  // unconditional: `ahead` then needs no merge of two versions
    if (b * 16 > lim) {   // every later position is masked as well
      for (int bb = b; bb < b1; ++bb) {
        const int s = bb * 16 + col;
        if (g == 0 && s < p.S) srow[s] = -INFINITY;
      }
      return false;
    }
    const int s = b * 16 + col;
    const bool two = kc.kmax < kTwoPieceLimit;
    const bool fits = (int64_t)qmax * kc.kmax * kIdxDim < (1LL << 31);
    if constexpr (NQP == 2) {
      if (two && fits) {
        i32x4 P00[NHB], X[NHB], P11[NHB];
        float G = 0.f;
#pragma unroll
        for (int hb = 0; hb < NHB; ++hb) two_piece(kc.k, hb, P00[hb], X[hb], P11[hb]);
#pragma unroll
        for (int hb = 0; hb < NHB; ++hb) epilogue(P00[hb], X[hb], P11[hb], hb, G);
        finish(G, kc.cs, s);
        return true;
      }
    }
    general(kc, b, s, two);
    return true;
  };
  for (int b = b0; b < b1; b += 3) {
    if (!step(b, ka, kc3) || b + 1 >= b1) break;
    if (!step(b + 1, kb, ka) || b + 2 >= b1) break;
    if (!step(b + 2, kc3, kb)) break;
  }
}

// Instruction groups for the scheduler (__builtin_amdgcn_sched_group_barrier
// masks: 0x002 VALU, 0x008 MFMA, 0x020 vector memory read, 0x040 write): NM
// MFMAs, each followed by NV VALU instructions.
template <int NM, int NV>
__device__ __forceinline__ void mfma_valu_groups() {
#pragma unroll
  for (int i = 0; i < NM; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x002, NV, 0);
  }
}

// Scores of token t over the blocks [b0, b1) when every block of the range
// takes the two-piece int32 path, for NHB >= 2: the same exact D and the same
// rounding order as score_range, from three piece products instead of four.
//
// With the pieces of every value below 2^14 in [0, 127] and of one sign,
// (q1 - q0) and (k0 - k1) fit int8 (the prep kernel writes them as planes).
// With P00 = q0.k0, P11 = q1.k1 and the cross term X = q0.k1 + q1.k0,
// (q1 - q0).(k0 - k1) = X - P00 - P11, so the chain
//   C3 = P00 + (q1 - q0).(k0 - k1) = X - P11
// gives D = P00 + 2^7 X + 2^14 P11 = ((C3 + 129 P11) << 7) + P00:
// six MFMAs per head block (C3's chain starts from P00's result) and two
// integer instructions per element (v_mad_i32_i24: |P11| < 2^23; the
// arithmetic is modulo 2^32 and D itself fits int32).  The int8 MFMA path
// is bound by the chip's power limit, not by issue: fewer MFMAs are faster.
//
// Two waves share the token's range (the two waves of one SIMD: one of
// them is issued first, and with fixed halves it would finish long before
// the other, which then runs alone): each claims chunks of six blocks from
// the pair's counter in LDS (`claim`, counting blocks from b0), one chunk
// ahead, until the range is used up.  Claims only grow, so every wave ends.
//
// Software-pipelined over the wave's sequence of head blocks j: the six
// MFMAs of head block j are issued between the epilogue instructions of head
// block j - 2, whose accumulators are complete by then; the pipeline runs
// on across chunk boundaries.  A chunk holds six blocks, so the three
// accumulator sets (j mod 3), the three operand buffers (fetched two blocks
// ahead), the group sums G[slot mod 2] and the pair scales, indexed by a
// block's slot in its chunk, all have static indices.  A pair of blocks
// shares one reduction over the four lane groups (a permlane16 swap of the
// two blocks' sums, a permlane32 swap, two adds: lane groups 0 and 1 end
// with blocks q and q + 1), one scale load and one store.
//
// Loads and stores go through buffer descriptors with scalar block offsets;
// scale loads and score stores carry the position in the per-lane offset,
// which the descriptor's bound checks (positions past S read 0 and are not
// stored; an offset of 2^31 is past every bound).  No per-block bound is
// loaded: a wave-uniform loaded value is moved to a scalar register right
// after its load, a wait that would tie each prefetch to its own step.
template <int NHB>
__device__ __forceinline__ void score_range_fast(const IndexerParams &p, const uint32_t *lut, int t,
                                                 int b0, int b1, int *claim, bool lead) {
#pragma clang fp contract(off)
  static_assert(NHB >= 2, "the epilogue runs two head blocks behind");
  const int lane = threadIdx.x & 63;
  const int col = lane & 15, g = lane >> 4;
  const int lim = p.limit[t];
  const int nkb = (p.S + 15) >> 4;
  const auto krs = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(p.k_pieces), 0,
                                                     nkb * kBlockBytes, kBufferFlags);
  const auto srs = __builtin_amdgcn_make_buffer_rsrc(p.k_cs, 0, p.S * 4, kBufferFlags);
  const auto ors = __builtin_amdgcn_make_buffer_rsrc(p.scores + (int64_t)t * p.S, 0, p.S * 4,
                                                     kBufferFlags);
  constexpr uint32_t kDropped = 0x80000000u;  // S * 4 < 2^31
  const uint32_t pair4 = (uint32_t)((g & 1) * 16 + col) * 4;  // lane's position in a pair, bytes
  uint32_t sh7;
  asm volatile("s_mov_b32 %0, 7" : "=s"(sh7));

  // blocks [b0, bend) hold a position at or below the causal limit; every
  // position of the blocks before bend - 1 is below it
  const int bend = min(b1, max(b0, (lim >> 4) + 1));
  if (lead)
    for (int b = bend; b < b1; ++b)
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(-INFINITY), ors,
                                            g == 0 ? col * 4 + b * 64 : kDropped, 0, 0);
  // first block of the next chunk of six the pair has not claimed yet
  auto claim_chunk = [&]() {
    int c = 0;
    if (lane == 0) c = atomicAdd(claim, 6);
    return b0 + __builtin_amdgcn_readfirstlane(c);
  };
  int B = claim_chunk();  // the current chunk
  if (B >= bend) return;
  int N = claim_chunk();  // the next one

  // A operands [hb][q0, q1, q1 - q0][k-step]
  i32x4 qa[NHB][3][2];
  {
    const int planes[3] = {0, 1, 4};
#pragma unroll
    for (int hb = 0; hb < NHB; ++hb) q_operands<3>(p, lut, t, hb, planes, qa[hb]);
  }
  float wl[NHB][4];
  const float *wsrc = p.w + (int64_t)t * p.Hi + g * (p.Hi >> 2);
#pragma unroll
  for (int hb = 0; hb < NHB; ++hb)
#pragma unroll
    for (int i = 0; i < 4; ++i) wl[hb][i] = wsrc[4 * hb + i];

  // B operands [k0, k1, k0 - k1][k-step] of a block (k slots 0, 1, 2)
  i32x4 kbuf[3][3][2];
  auto fetch_k = [&](int b, i32x4 (&k)[3][2]) {
    b = min(b, bend - 1);
#pragma unroll
    for (int pl = 0; pl < 3; ++pl)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
        k[pl][ks] = __builtin_bit_cast(
            i32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, lane * 16,
                                                         b * kBlockBytes + (pl * 2 + ks) * kChunk, 0));
  };
  // c_s of the pair starting at block q: lane groups g and g ^ 2 hold block q + (g & 1)
  auto fetch_cs = [&](int q) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(srs, pair4 + q * 64, 0, 0));
  };
  struct Acc {
    i32x4 P00, C3, P11;
  };
  Acc acc[3];
  auto mm = [&](const i32x4 (&k)[3][2], int hb, Acc &a) {
    const i32x4 z = {0, 0, 0, 0};
    a.P00 = mfma(qa[hb][0][1], k[0][1], mfma(qa[hb][0][0], k[0][0], z));
    a.P11 = mfma(qa[hb][1][1], k[1][1], mfma(qa[hb][1][0], k[1][0], z));
    a.C3 = mfma(qa[hb][2][1], k[2][1], mfma(qa[hb][2][0], k[2][0], a.P00));
  };
  // D = ((C3 + 129 P11) << 7) + P00, then the ReLU, the conversion and the
  // head's fused multiply-add into the group sum
  auto epi = [&](const Acc &a, int hb, float &G) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t hi = (uint32_t)__mul24(a.P11[i], 129) + (uint32_t)a.C3[i];
      const int D = (int)((hi << sh7) + (uint32_t)a.P00[i]);
      G = __builtin_fmaf(wl[hb][i], (float)max(D, 0), G);
    }
  };
  float G[2] = {0.f, 0.f};  // the lane's group sums of the current pair's blocks
  // the pair starting at block q: (G0 + G1) + (G2 + G3) of both blocks, times
  // c_s, stored by lane groups 0 and 1; `last` masks the positions past the
  // causal limit and a second block at or past bend
  auto store_pair = [&](int q, float cs, bool last) {
    auto x = __builtin_amdgcn_permlane16_swap(__float_as_uint(G[0]), __float_as_uint(G[1]), false, false);
    const float a = __uint_as_float(x[0]) + __uint_as_float(x[1]);  // rows: G0+G1 | G2+G3 of q, q+1
    auto y = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(a), false, false);
    const float total = __uint_as_float(y[0]) + __uint_as_float(y[1]);  // block q + (g & 1)
    float v = total * cs;
    const int blk = q + (g & 1);
    uint32_t off = g < 2 ? pair4 + q * 64 : kDropped;
    if (last) {
      if (blk * 16 + col > lim) v = -INFINITY;
      if (blk >= bend) off = kDropped;
    }
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), ors, off, 0, 0);
  };

  float cs_pair[3];  // scales of the pairs starting at slots 0, 2, 4
  fetch_k(B, kbuf[0]);
  fetch_k(B + 1, kbuf[1]);
  fetch_k(B + 2, kbuf[2]);
  cs_pair[0] = fetch_cs(B);
  {  // block B (slot 0; the stages fetch two blocks ahead)
    float Gc = 0.f;
#pragma unroll
    for (int hb = 0; hb < NHB; ++hb) {
      if (hb >= 2) epi(acc[(hb - 2) % 3], hb - 2, Gc);
      mm(kbuf[0], hb, acc[hb % 3]);
    }
    G[0] = Gc;
  }
  // block b in slot SLOT of its chunk: fetch the block two ahead (`ahead`:
  // past the chunk, in the next one), finish the previous block (and, for an
  // even SLOT, store the pair before it, which starts at `pair`), issue block
  // b's MFMAs
  auto stage = [&](int b, auto slot_c, int ahead, int pair) {
    constexpr int SLOT = decltype(slot_c)::value;
    constexpr bool kEven = (SLOT & 1) == 0;
    fetch_k(ahead, kbuf[(SLOT + 2) % 3]);
    if constexpr (kEven) {
      cs_pair[SLOT / 2] = fetch_cs(b);
      __builtin_amdgcn_sched_group_barrier(0x020, 7, 0);
    } else {
      __builtin_amdgcn_sched_group_barrier(0x020, 6, 0);
    }
    float Gc = 0.f;
#pragma unroll
    for (int hb = 0; hb < NHB; ++hb) {
      const int j = SLOT * NHB + hb;
      if (hb < 2) {
        epi(acc[(j + 1) % 3], hb + NHB - 2, G[(SLOT + 1) & 1]);
        if (kEven && hb == 1) store_pair(pair, cs_pair[(SLOT / 2 + 2) % 3], false);
      } else {
        epi(acc[(j + 1) % 3], hb - 2, Gc);
      }
      mm(kbuf[SLOT % 3], hb, acc[j % 3]);
      if (kEven && hb == 1) {
        mfma_valu_groups<6, 4>();
        __builtin_amdgcn_sched_group_barrier(0x040, 1, 0);
      } else {
        mfma_valu_groups<6, 3>();
      }
      // the pipeline above pairs each head block's MFMAs with finished
      // accumulators: nothing moves between head blocks (an MFMA moved
      // earlier would wait for operands loaded in the same iteration)
      __builtin_amdgcn_sched_barrier(0);
    }
    G[SLOT & 1] = Gc;
  };
  // after the wave's last block (slot SLOT of its chunk): its last two head
  // blocks, then its pair
  auto drain = [&](auto slot_c, int last) {
    constexpr int SLOT = decltype(slot_c)::value;
    constexpr int j = SLOT * NHB + NHB - 1;
    epi(acc[(j + 2) % 3], NHB - 2, G[SLOT & 1]);
    epi(acc[j % 3], NHB - 1, G[SLOT & 1]);
    store_pair(last - (SLOT & 1), cs_pair[SLOT / 2], true);
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  using S3 = std::integral_constant<int, 3>;
  using S4 = std::integral_constant<int, 4>;
  using S5 = std::integral_constant<int, 5>;
  // blocks 1 .. 5 of a full chunk B, then block 0 of the next chunk N
  while (B + 6 <= bend && N < bend) {
    const int N2 = claim_chunk();
    stage(B + 1, S1{}, B + 3, 0);
    stage(B + 2, S2{}, B + 4, B);
    stage(B + 3, S3{}, B + 5, 0);
    stage(B + 4, S4{}, N, B + 2);
    stage(B + 5, S5{}, N + 1, 0);
    stage(N, S0{}, N + 2, B + 4);
    B = N;
    N = N2;
  }
  // the wave's last chunk: blocks 1 .. rest (the operand fetches past it are
  // clamped to bend - 1 and unused)
  const int rest = min(bend, B + 6) - 1 - B;
  if (rest > 0) stage(B + 1, S1{}, B + 3, 0);
  if (rest > 1) stage(B + 2, S2{}, B + 4, B);
  if (rest > 2) stage(B + 3, S3{}, B + 5, 0);
  if (rest > 3) stage(B + 4, S4{}, B + 6, B + 2);
  if (rest > 4) stage(B + 5, S5{}, B + 7, 0);
  switch (rest) {
    case 0: drain(S0{}, B); break;
    case 1: drain(S1{}, B + 1); break;
    case 2: drain(S2{}, B + 2); break;
    case 3: drain(S3{}, B + 3); break;
    case 4: drain(S4{}, B + 4); break;
    default: drain(S5{}, B + 5); break;
  }
}

template <int NHB>
__global__ __launch_bounds__(kScoreWaves * 64) void dsa_idx_score_kernel(IndexerParams p) {
  // two waves per token: slot = the token's place in the workgroup, member
  // 0 or 1 (waves w and w + tpw, which the hardware places on one SIMD)
  __shared__ int claim[kScoreWaves / 2];
  __shared__ uint32_t lut[256];  // code -> its pieces (piece_word)
  const int tpw = blockDim.x >> 7;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int slot = wave % tpw, member = wave / tpw;
  if (threadIdx.x < kScoreWaves / 2) claim[threadIdx.x] = 0;
  for (int i = threadIdx.x; i < 256; i += blockDim.x) lut[i] = piece_word(i);
  __syncthreads();
  const int t = blockIdx.y * tpw + slot;
  const int nkb = (p.S + 15) >> 4;
  const int b0 = blockIdx.x * p.blocks_per_wg;
  const int b1 = min(nkb, b0 + p.blocks_per_wg);
  if (t >= p.T || b0 >= b1) return;
  // the general paths split the range in halves
  const int mid = b0 + (b1 - b0 + 1) / 2;
  const int h0 = member == 0 ? b0 : mid, h1 = member == 0 ? mid : b1;
  const int qmax = q_magnitude_bound(p, t);
  if (qmax >= kTwoPieceLimit) {
    if (h0 < h1) score_range<NHB, 3>(p, lut, t, h0, h1, qmax);
    return;
  }
  // the range's largest block bound decides whether every block takes the
  // three-product path
  if constexpr (NHB >= 2) {
    const int lane = threadIdx.x & 63;
    int rmax = 0;
    for (int b = b0 + lane; b < b1; b += 64) rmax = max(rmax, p.k_max[b]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) rmax = max(rmax, __shfl_xor(rmax, o));
    rmax = __builtin_amdgcn_readfirstlane(rmax);
    const bool descriptors_fit = (int64_t)nkb * kBlockBytes < (1LL << 31);
    if (rmax < kTwoPieceLimit && (int64_t)qmax * rmax * kIdxDim < (1LL << 31) && descriptors_fit) {
      score_range_fast<NHB>(p, lut, t, b0, b1, &claim[slot], member == 0);
      return;
    }
  }
  if (h0 < h1) score_range<NHB, 2>(p, lut, t, h0, h1, qmax);
}

// ---- top-k ---------------------------------------------------------------

__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f == 0.f ? 0.f : f);  // -0 -> +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ void emit_pos(const IndexerParams &p, int t, int32_t *out, int pos,
                                         int rank) {
  int v = pos;
  if (p.block_table != nullptr) {
    const int32_t page = p.block_table[(int64_t)t * p.bt_stride + pos / p.page_size];
    v = page * p.page_size + pos % p.page_size;
  }
  out[rank] = v;
}

// Inclusive prefix sum over the 64 lanes of a wave: row shifts within rows
// of 16 lanes, then the row totals carried with the row broadcasts (gfx9
// wave64 DPP; lanes without a source add 0).
__device__ __forceinline__ int wave_inclusive_sum(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15 -> rows 1, 3
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31 -> rows 2, 3
  return v;
}

// Exclusive prefix sums of (a, b) over the 1024 threads of the block; the
// totals go to *ta, *tb.  Wave sums, then wave 0 scans the 16 wave totals.
__device__ int2 block_exclusive_scan2(int a, int b, int2 *scratch, int *ta, int *tb) {
  constexpr int kWaves = kTopkThreads / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int x = wave_inclusive_sum(a), y = wave_inclusive_sum(b);
  if (lane == 63) scratch[wave] = make_int2(x, y);
  __syncthreads();
  if (wave == 0) {
    const int2 w = lane < kWaves ? scratch[lane] : make_int2(0, 0);
    const int ix = wave_inclusive_sum(w.x), iy = wave_inclusive_sum(w.y);
    if (lane < kWaves) scratch[lane] = make_int2(ix - w.x, iy - w.y);
    if (lane == kWaves - 1) scratch[kWaves] = make_int2(ix, iy);
  }
  __syncthreads();
  const int2 base = scratch[wave];
  *ta = scratch[kWaves].x;
  *tb = scratch[kWaves].y;
  __syncthreads();
  return make_int2(base.x + x - a, base.y + y - b);
}

// After one pass's histogram is in tot[]: the digit that holds the
// `need`-th largest key among those matching the prefix.  Run by wave 0.
__device__ __forceinline__ void pick_digit(const uint32_t *tot, uint32_t prefix, uint32_t mask,
                                           int shift, int need, uint32_t *s_prefix,
                                           uint32_t *s_mask, int *s_need) {
  // Lane l owns bins b0 .. b0+3 with b0 = 4*(63 - l), so the bins above
  // its own belong to lanes 0..l-1: their count is an exclusive prefix sum.
  const int l = threadIdx.x;
  const int b0 = 4 * (63 - l);
  const uint32_t c0 = tot[b0], c1 = tot[b0 + 1], c2 = tot[b0 + 2], c3 = tot[b0 + 3];
  const uint32_t local = c0 + c1 + c2 + c3;
  uint32_t cum = (uint32_t)wave_inclusive_sum((int)local) - local;  // keys in the bins above
  const uint32_t cs[4] = {c0, c1, c2, c3};
#pragma unroll
  for (int b = 3; b >= 0; --b) {
    if ((int)cum < need && (int)(cum + cs[b]) >= need) {
      *s_prefix = prefix | ((uint32_t)(b0 + b) << shift);
      *s_mask = mask | (255u << shift);
      *s_need = need - (int)cum;
    }
    cum += cs[b];
  }
}

// v_writelane_b32 (the LLVM intrinsic; the compiler inserts the wait states
// it needs after the VALU write of its SGPR source).
extern "C" __device__ int amdgcn_writelane(int value, int lane, int old) __asm("llvm.amdgcn.writelane.i32");

// Survivors of the first two radix passes that the register top-k ranks
// directly; more take two more passes.
constexpr int kMaxSurvivors = 256;

// Shared state of one top-k workgroup (KEYS = positions it holds).  One
// space serves the radix histograms and then the selected positions by
// rank.  The bitmaps hold one bit per position: 64-bit word e*16 + w covers
// positions e*1024 + 64w .. +63, i.e. the keys e of wave w's 64 lanes.
template <int KEYS>
struct TopkShared {
  union {
    uint32_t hist[2][kHistCopies * kHistPitch];  // one per radix pass of the register top-k
    int32_t pos[KEYS];
  };
  uint64_t bits[KEYS / 64 > 0 ? KEYS / 64 : 1];    // selected
  uint64_t eqbits[KEYS / 64 > 0 ? KEYS / 64 : 1];  // ties of the k-th key
  uint2 cand[kMaxSurvivors];                       // (key, position), any order
  uint32_t tot[256];
  int2 scan[kTopkThreads / 64 + 1];
  uint32_t prefix, mask;
  int need, n_cand;
};

// Rows with at most topk candidates: every candidate, then -1.
// Number of candidate positions of row t: s is one iff s <= causal_limit[t]
// and s < S.  Compared before adding one, so a limit of INT32_MAX (no limit)
// does not wrap to a negative count.
__device__ __forceinline__ int candidates(const IndexerParams &p, int t) {
  const int lim = p.limit[t];
  return lim >= p.S - 1 ? p.S : max(0, lim + 1);
}

__device__ __forceinline__ bool take_all(const IndexerParams &p, int t, int32_t *out, int n) {
  if (n > p.topk) return false;
  for (int i = threadIdx.x; i < p.topk; i += kTopkThreads) {
    if (i < n) emit_pos(p, t, out, i, i);
    else out[i] = -1;
  }
  return true;
}

// One radix pass: histogram of the digit at `shift` over the keys matching
// the prefix (everything else is counted in the spare bin 256 of each copy,
// so the atomics need no branch), then the digit of the need-th largest.
// for_keys(f) calls f(key, is_candidate) for each of this thread's keys.
// `phantom` keys of value 0 that are not candidates were counted too (they
// sit in bin 0 while the prefix is 0) and are taken out of that bin.
template <typename Shared, typename ForKeys>
__device__ __forceinline__ void radix_pass(Shared &sh, int shift, ForKeys for_keys,
                                           uint32_t &prefix, uint32_t &mask, int &need,
                                           int phantom = 0) {
  for (int i = threadIdx.x; i < kHistCopies * kHistPitch; i += kTopkThreads) sh.hist[0][i] = 0;
  __syncthreads();
  uint32_t *myhist = sh.hist[0] + (threadIdx.x & (kHistCopies - 1)) * kHistPitch;
  const uint32_t pf = prefix, mk = mask;
  for_keys([&](uint32_t key, bool cand) {
    const uint32_t bin = (cand && (key & mk) == pf) ? ((key >> shift) & 255u) : 256u;
    atomicAdd(&myhist[bin], 1u);
  });
  __syncthreads();
  if (threadIdx.x < 256) {
    uint32_t c = 0;
#pragma unroll 8
    for (int j = 0; j < kHistCopies; ++j) c += sh.hist[0][j * kHistPitch + threadIdx.x];
    if (threadIdx.x == 0 && prefix == 0) c -= (uint32_t)phantom;
    sh.tot[threadIdx.x] = c;
  }
  __syncthreads();
  if (threadIdx.x < 64) pick_digit(sh.tot, prefix, mask, shift, need, &sh.prefix, &sh.mask, &sh.need);
  __syncthreads();
  prefix = sh.prefix;
  mask = sh.mask;
  need = sh.need;
}

// Key of the positions past a row's candidates in the register top-k: the
// buffer load reads them as 0.0.
constexpr uint32_t kPhantomKey = 0x80000000u;

// One radix pass over the register-resident keys of a row, into histogram
// `hist`: with `zeroed` the caller zeroed it and passed a barrier since,
// otherwise the pass zeroes it first.  Under prefix pf (the digits above
// `shift` fixed so far) a key's digit is (k - pf) >> shift when it matches the
// prefix (then below 256) and at least 256 otherwise.  The first pass (no
// prefix) counts every key, min(., 256) keeping the branch out; later passes
// issue atomics only for the keys under the prefix.  The copies are added by
// all threads, four per bin (eight copies each, then a quad sum).  The
// `phantom` copies of kPhantomKey are taken out of their bin.
template <int EPT, typename Shared>
__device__ __forceinline__ void radix_pass_regs(Shared &sh, uint32_t *hist, bool zeroed, int shift,
                                                const uint32_t (&key)[EPT], uint32_t &prefix,
                                                uint32_t &mask, int &need, int phantom) {
  static_assert(kTopkThreads == 4 * 256, "four threads per bin in the copy sum");
  if (!zeroed) {
    for (int i = threadIdx.x; i < kHistCopies * kHistPitch; i += kTopkThreads) hist[i] = 0;
    __syncthreads();
  }
  uint32_t *myhist = hist + (threadIdx.x & (kHistCopies - 1)) * kHistPitch;
  const uint32_t pf = prefix;
  if (mask == 0) {  // first pass: every key counts
#pragma unroll
    for (int e = 0; e < EPT; ++e) atomicAdd(&myhist[min((key[e] - pf) >> shift, 256u)], 1u);
  } else {  // later passes: only the keys under the prefix (few) issue an atomic
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const uint32_t d = (key[e] - pf) >> shift;
      if (d < 256u) atomicAdd(&myhist[d], 1u);
    }
  }
  __syncthreads();
  {
    const int bin = threadIdx.x >> 2, q = threadIdx.x & 3;
    constexpr int kPer = kHistCopies / 4;
    uint32_t c = 0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) c += hist[(q * kPer + j) * kHistPitch + bin];
    c += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)c, 0xb1, 0xf, 0xf, false);  // quad_perm [1,0,3,2]
    c += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)c, 0x4e, 0xf, 0xf, false);  // quad_perm [2,3,0,1]
    if (bin == (int)min((kPhantomKey - pf) >> shift, 256u)) c -= (uint32_t)phantom;
    if (q == 0) sh.tot[bin] = c;
  }
  __syncthreads();
  if (threadIdx.x < 64) pick_digit(sh.tot, prefix, mask, shift, need, &sh.prefix, &sh.mask, &sh.need);
  __syncthreads();
  prefix = sh.prefix;
  mask = sh.mask;
  need = sh.need;
}

template <int EPT>
__global__ __launch_bounds__(kTopkThreads) void dsa_idx_topk_kernel(IndexerParams p) {
  static_assert(EPT <= 32, "one 32-bit bitmap word per thread at most");
  constexpr int KEYS = EPT * kTopkThreads;
  static_assert(KEYS <= 32768, "survivor ranks pack positions in 15 bits");
  constexpr int kWaves = kTopkThreads / 64;
  __shared__ TopkShared<KEYS> sh;
  const int t = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // known uniform: scalar masks
  const float *row = p.scores + (int64_t)t * p.S;
  int32_t *out = p.out + (int64_t)t * p.topk;
  const int n = candidates(p, t);  // candidates 0..n-1
  if (take_all(p, t, out, n)) return;               // n > topk >= 1 below

  // Key e of this thread is position e*1024 + tid (coalesced), so the 64
  // lanes of a wave hold 64 consecutive positions of every e.  A buffer load
  // over the n candidates needs one 32-bit offset register for all 32 loads
  // (kept in flight together) and reads the positions past n as 0.0: those
  // `phantom` keys are taken out of the histograms and masked out of the
  // selection by position, which is uniform per wave and e.  Adding +0.0
  // turns -0.0 into +0.0; the key orders the scores as unsigned integers.
  uint32_t key[EPT];
  {
    const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(row), 0, n * 4, 0x00020000);
#pragma unroll
    for (int e = 0; e < EPT; ++e)
      key[e] = __builtin_amdgcn_raw_buffer_load_b32(rs, tid * 4, e * kTopkThreads * 4, 0);
  }
  const int phantom = KEYS - n;
  if (tid == 0) sh.n_cand = 0;  // ordered before its use by the passes' barriers
  // both passes' histograms are zeroed while the key loads are in flight
  for (int i = tid; i < 2 * kHistCopies * kHistPitch; i += kTopkThreads) (&sh.hist[0][0])[i] = 0;
  __syncthreads();
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const uint32_t u = __builtin_bit_cast(uint32_t, __builtin_bit_cast(float, key[e]) + 0.0f);
    key[e] = u ^ ((uint32_t)((int32_t)u >> 31) | 0x80000000u);
  }

  // Two passes: the k-th largest key lies in the 16-bit bin `prefix`; keys
  // above the bin are all taken and `need` more come from its survivors.
  uint32_t prefix = 0, mask = 0;
  int need = p.topk, unused;
#pragma unroll 1
  for (int shift = 24; shift >= 16; shift -= 8)
    radix_pass_regs(sh, sh.hist[shift == 24 ? 0 : 1], true, shift, key, prefix, mask, need, phantom);

  // Selection as a position bitmap, built from ballots of the registers
  // (64-bit word e*16 + wave holds key e of the wave's lanes: lane 2e + h
  // collects half h and one store per lane writes them).  Positions past n
  // are masked out when the words are read.  Waves holding survivors of the
  // bin list them (key, position) for an exact ranking.
  uint32_t *bits32 = (uint32_t *)sh.bits;  // word w: positions 32w .. 32w+31
  {
    const uint32_t hi = prefix | 0xffffu;  // keys above the bin
    uint32_t bw = 0;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const uint64_t ab = __ballot(key[e] > hi);
      const uint64_t sb = __ballot(key[e] >= prefix) & ~ab;  // keys in the bin
      bw = (uint32_t)amdgcn_writelane((int)(uint32_t)ab, 2 * e, (int)bw);
      bw = (uint32_t)amdgcn_writelane((int)(uint32_t)(ab >> 32), 2 * e + 1, (int)bw);
      if (sb != 0) {  // uniform
        int o = 0;
        if (lane == 0) o = atomicAdd(&sh.n_cand, __popcll(sb));
        o = __builtin_amdgcn_readfirstlane(o) +
            __builtin_amdgcn_mbcnt_hi((uint32_t)(sb >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)sb, 0));
        if (((sb >> lane) & 1) && o < kMaxSurvivors)
          sh.cand[o] = make_uint2(key[e], (uint32_t)(e * kTopkThreads + tid));
      }
    }
    if (lane < 2 * EPT) bits32[((lane >> 1) * kWaves + wave) * 2 + (lane & 1)] = bw;
  }
  __syncthreads();
  const int n_surv = sh.n_cand;
  if (n_surv <= kMaxSurvivors) {  // uniform
    // Rank: key descending, position ascending, among the survivors below n
    // (the list may hold positions past n).  Four lanes per survivor each
    // count the survivors ahead of it in a quarter of the list, and two DPP
    // quad swaps add the counts; the first `need` are marked.
    {
      const int i = tid >> 2, q = tid & 3;
      if (i < ((n_surv + 15) & ~15)) {  // whole waves
        const uint2 me = sh.cand[min(i, n_surv - 1)];
        int r = 0;
        // four reads in flight per step (entries past the list count nothing)
        for (int j0 = q; j0 < n_surv; j0 += 16) {
          uint2 c[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) c[u] = sh.cand[min(j0 + 4 * u, kMaxSurvivors - 1)];
#pragma unroll
          for (int u = 0; u < 4; ++u)
            r += j0 + 4 * u < n_surv && (int)c[u].y < n &&
                 (c[u].x > me.x || (c[u].x == me.x && c[u].y < me.y));
        }
        r += __builtin_amdgcn_update_dpp(0, r, 0xb1, 0xf, 0xf, false);  // quad_perm [1,0,3,2]
        r += __builtin_amdgcn_update_dpp(0, r, 0x4e, 0xf, 0xf, false);  // quad_perm [2,3,0,1]
        if (q == 0 && i < n_surv && (int)me.y < n && r < need)
          atomicOr(&bits32[me.y >> 5], 1u << (me.y & 31));
      }
    }
    __syncthreads();
  } else {
    // Many keys share the bin: two more passes pin the k-th key itself;
    // keys above it are taken, and `need` of its ties, lowest positions first.
#pragma unroll 1
    for (int shift = 8; shift >= 0; shift -= 8)
      radix_pass_regs(sh, sh.hist[0], false, shift, key, prefix, mask, need, phantom);
    // (Ties past n sit after every real position and `need` counts real
    // ones only, so they are never taken; the masking below clears the rest.)
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const uint64_t gb = __ballot(key[e] > prefix);
      const uint64_t qb = __ballot(key[e] == prefix);
      if (lane == 0) {
        sh.bits[e * kWaves + wave] = gb;
        sh.eqbits[e * kWaves + wave] = qb;
      }
    }
    __syncthreads();
    uint32_t eq = tid < KEYS / 32 ? ((const uint32_t *)sh.eqbits)[tid] : 0u;
    int tot_eq;
    const int2 ex = block_exclusive_scan2(__builtin_popcount(eq), 0, sh.scan, &tot_eq, &unused);
    uint32_t take = 0;
    for (int left = need - ex.x; left > 0 && eq != 0; --left) {
      take |= eq & (~eq + 1);
      eq &= eq - 1;
    }
    if (take != 0) bits32[tid] |= take;  // this thread's own word
  }

  // Output ranks in position order: thread tid owns bitmap word tid; the
  // selected positions go to LDS by rank (the scan's barriers order this
  // after every bitmap read), then each thread maps up to four of them
  // through the block table with the loads issued together and stores them
  // coalesced.
  const int nw = n - tid * 32;  // this word's positions below n
  uint32_t sel = tid < KEYS / 32 ? bits32[tid] : 0u;
  sel &= nw >= 32 ? ~0u : (nw <= 0 ? 0u : (1u << nw) - 1u);
  int n_sel;
  const int2 rx = block_exclusive_scan2(__builtin_popcount(sel), 0, sh.scan, &n_sel, &unused);
  int o = rx.x;
  while (sel != 0) {
    const int e = __builtin_ctz(sel);
    sel &= sel - 1;
    sh.pos[o++] = tid * 32 + e;
  }
  __syncthreads();
  for (int r0 = tid; r0 < p.topk; r0 += 4 * kTopkThreads) {
    int v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = sh.pos[min(r0 + u * kTopkThreads, p.topk - 1)];
    if (p.block_table != nullptr) {
      const int32_t *bt = p.block_table + (int64_t)t * p.bt_stride;
      int page[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) page[u] = bt[v[u] / p.page_size];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = page[u] * p.page_size + v[u] % p.page_size;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (r0 + u * kTopkThreads < p.topk) out[r0 + u * kTopkThreads] = v[u];
  }
}

// Rows longer than the register kernel holds: the same selection, reading
// the row from memory in every pass.
__global__ __launch_bounds__(kTopkThreads) void dsa_idx_topk_stream_kernel(IndexerParams p) {
  __shared__ TopkShared<0> sh;
  const int t = blockIdx.x;
  const float *row = p.scores + (int64_t)t * p.S;
  int32_t *out = p.out + (int64_t)t * p.topk;
  const int n = candidates(p, t);
  if (take_all(p, t, out, n)) return;

  uint32_t prefix = 0, mask = 0;
  int need = p.topk;
  for (int shift = 24; shift >= 0; shift -= 8)
    radix_pass(sh, shift,
               [&](auto f) {
                 for (int i = threadIdx.x; i < n; i += kTopkThreads) f(order_key(row[i]), true);
               },
               prefix, mask, need);
  // ordered compaction: thread i owns positions [i*chunk, (i+1)*chunk)
  const int chunk = (n + kTopkThreads - 1) / kTopkThreads;
  const int c0 = min(n, (int)threadIdx.x * chunk), c1 = min(n, c0 + chunk);
  int n_gt = 0, n_eq = 0;
  for (int i = c0; i < c1; ++i) {
    const uint32_t key = order_key(row[i]);
    n_gt += key > prefix;
    n_eq += key == prefix;
  }
  int tot_gt, tot_eq;
  const int2 ex = block_exclusive_scan2(n_gt, n_eq, sh.scan, &tot_gt, &tot_eq);
  int o = ex.x + min(ex.y, need);
  int eq_left = need - ex.y;
  for (int i = c0; i < c1; ++i) {
    const uint32_t key = order_key(row[i]);
    bool sel = key > prefix;
    if (key == prefix) {
      sel = eq_left > 0;
      --eq_left;
    }
    if (sel) emit_pos(p, t, out, i, o++);
  }
}

// ---- quantise-on-append into the paged K cache ---------------------------

// e4m3fn code of x (finite, |x| <= 448), rounded to nearest, ties to even.
__device__ __forceinline__ uint32_t e4m3_encode(float x) {
  const uint32_t sign = (__float_as_uint(x) >> 24) & 0x80u;
  const float a = fabsf(x);
  uint32_t code;
  if (a < 0x1p-6f) {  // zero and the subnormals: multiples of 2^-9 (8 = the smallest normal)
    code = (uint32_t)__builtin_rintf(a * 512.0f);
  } else {            // 3 mantissa bits, ties to even; exponent rebiased 127 -> 7
    const uint32_t m = __float_as_uint(a);
    const uint32_t r = m + 0x7ffffu + ((m >> 20) & 1u);
    code = (((r >> 23) - 120u) << 3) | ((r >> 20) & 7u);
  }
  return sign | code;
}

// One wave per token: lane l quantises elements 2l, 2l+1.
__global__ __launch_bounds__(256) void dsa_k_append_kernel(KAppendParams p) {
  const int lane = threadIdx.x & 63;
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= p.n) return;
  const int slot = p.slots[i];
  if (slot < 0 || slot >= p.num_slots) return;
  const uint32_t pair = *(const uint32_t *)(p.k + (int64_t)i * p.k_stride + 2 * lane);
  const float x0 = __uint_as_float(pair << 16), x1 = __uint_as_float(pair & 0xffff0000u);
  float amax = fmaxf(fabsf(x0), fabsf(x1));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  const float scale = fmaxf(amax, 1e-4f) / 448.0f;
  const float y0 = fminf(fmaxf(x0 / scale, -448.0f), 448.0f);
  const float y1 = fminf(fmaxf(x1 / scale, -448.0f), 448.0f);
  const int pg = slot / p.page_size, off = slot - pg * p.page_size;
  uint8_t *page = p.cache + (int64_t)pg * p.page_size * kKTokenBytes;
  *(uint16_t *)(page + off * kIdxDim + 2 * lane) =
      (uint16_t)(e4m3_encode(y0) | (e4m3_encode(y1) << 8));
  if (lane == 0) *(float *)(page + p.page_size * kIdxDim + off * 4) = scale;
}

template <int NHB>
hipError_t launch_score(const IndexerParams &p, dim3 grid, dim3 block, hipStream_t stream) {
  hipLaunchKernelGGL(dsa_idx_score_kernel<NHB>, grid, block, 0, stream, p);
  return hipGetLastError();
}

template <int EPT>
hipError_t launch_topk(const IndexerParams &p, hipStream_t stream) {
  hipLaunchKernelGGL(dsa_idx_topk_kernel<EPT>, dim3(p.T), dim3(kTopkThreads), 0, stream, p);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_k_append(const KAppendParams &p, hipStream_t stream) {
  if (p.n == 0) return hipSuccess;
  hipLaunchKernelGGL(dsa_k_append_kernel, dim3((p.n + 3) / 4), dim3(256), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_indexer_prepare_k(const IndexerParams &p, hipStream_t stream) {
  if (p.k_blocks <= 0) return hipSuccess;
  const int prep_blocks = (p.k_blocks + kPrepThreads / 64 - 1) / (kPrepThreads / 64);
  hipLaunchKernelGGL(dsa_idx_prep_kernel, dim3(prep_blocks), dim3(kPrepThreads), 0, stream, p);
  return hipGetLastError();
}

hipError_t launch_indexer(const IndexerParams &pin, hipStream_t stream) {
  if (pin.T == 0) return hipSuccess;
  IndexerParams p = pin;
  const int nkb = (p.S + 15) / 16, nqb = p.Hi / 16;
  // the K planes, unless the call reads prepared ones (the q operands are
  // derived inside the score kernel)
  hipError_t e = launch_indexer_prepare_k(p, stream);
  if (e != hipSuccess) return e;
  if (p.S > 0) {
    // tokens per workgroup (two waves each) and 16-position blocks per
    // workgroup range, aiming at two waves per SIMD with at least 8 blocks
    // per wave
    const int tpw = std::min(p.T, kScoreWaves / 2);
    const int tgroups = (p.T + tpw - 1) / tpw;
    int bx = (kTargetScoreWaves + 2 * tpw * tgroups - 1) / (2 * tpw * tgroups);
    bx = std::min(bx, (nkb + 2 * kMinBlocksPerWave - 1) / (2 * kMinBlocksPerWave));
    bx = std::max(bx, 1);
    p.blocks_per_wg = (nkb + bx - 1) / bx;
    bx = (nkb + p.blocks_per_wg - 1) / p.blocks_per_wg;
    const dim3 grid(bx, tgroups), block(128 * tpw);
    switch (nqb) {
      case 1: e = launch_score<1>(p, grid, block, stream); break;
      case 2: e = launch_score<2>(p, grid, block, stream); break;
      case 3: e = launch_score<3>(p, grid, block, stream); break;
      default: e = launch_score<4>(p, grid, block, stream); break;
    }
    if (e != hipSuccess) return e;
  }
  if (p.topk > 0) {
    if (p.S <= kTopkThreads * 8) e = launch_topk<8>(p, stream);
    else if (p.S <= kTopkThreads * 16) e = launch_topk<16>(p, stream);
    else if (p.S <= kTopkThreads * kMaxRegEpt) e = launch_topk<kMaxRegEpt>(p, stream);
    else {
      hipLaunchKernelGGL(dsa_idx_topk_stream_kernel, dim3(p.T), dim3(kTopkThreads), 0, stream, p);
      e = hipGetLastError();
    }
  }
  return e;
}

}  // namespace dsa
