// dsa_indexer.hip -- lightning-indexer scores and per-row top-k for gfx950.
//
// Score (the structure of the reference's indexer_kernel,
// solution/triton/indexer_kernel.py:185-275: dequantise -> dot -> ReLU ->
// head weight -> sum over heads; BASELINE config 5 form):
//
//   score[t,s] = sum_h w[t,h] * relu(q[t,h,:] . k[s,:] * k_scale[s])
//
// with one exact rounding order, so the GPU reproduces the CPU oracle bit for
// bit: d = the exact dot of the e4m3fn values; a = fl32(fl32(d) * k_scale[s]);
// r = max(a, 0); v = fl32(w[t,h] * r); heads are summed in blocks of 16, in
// block order starting from 0, each block as (G0 + G1) + (G2 + G3) with
// G = ((v0 + v1) + v2) + v3 over 4 consecutive heads.  Positions beyond
// causal_limit[t] score -inf and are never selected.
//
// Exact dot on int8 MFMA.  Every finite e4m3fn value times 2^9 is an integer
// x with |x| <= 229376 (18 bits); x = p0 + 2^7 p1 + 2^14 p2 with signed 7-bit
// pieces (sign-magnitude split).  Then
//   d * 2^18 = sum_{a,b} 2^(7(a+b)) sum_j pq_a[j] pk_b[j]
// and each inner 128-term sum (|.| <= 128*127*127) is exact in the int32
// accumulator of v_mfma_i32_16x16x64_i8.  For |value| < 32 the third piece is
// zero and four piece products suffice; the combine is then exact in int32 when
// |P11| < 2^16 and the one int32 -> fp32 conversion rounds like fl32(d)
// (scaling by 2^-18 commutes with rounding; it is folded into k_scale).  Any
// other case takes an exact fp64 combine.  e4m3fn NaN codes (0x7f, 0xff) count
// as zero.
//
// Kernels:
//   dsa_idx_prep_q_kernel  one workgroup per token: q codes -> piece planes
//                          [T][Hi][3][128] int8 and the token's piece level.
//   dsa_idx_score_kernel   one workgroup per (256 positions, token group): the
//                          positions' k pieces stay in registers (B operands),
//                          each token's q pieces are staged in LDS (double
//                          buffered) and shared by the four waves.  Heads are
//                          the MFMA M dimension, positions N.
//   dsa_idx_topk_kernel    one workgroup per row: 4-pass radix select (8 bits
//                          per pass) of the k-th largest order-preserving key,
//                          then an ordered compaction that keeps every larger
//                          score and the lowest positions among the ties, in
//                          ascending position order (reference intent:
//                          indexer_kernel.py:289-343, strict '>' keeps the
//                          earlier index).
#include "../../include/dsa_abi.h"
#include "dsa_internal.h"

namespace dsa {
namespace {

typedef int i32x4 __attribute__((ext_vector_type(4)));

constexpr int kIdxDim = 128;
constexpr int kScoreSlots = 256;        // positions per score workgroup (4 waves x 4 x 16)
constexpr int kSlotBlocks = 4;          // 16-position MFMA blocks per wave
constexpr int kTokensPerGroup = 32;     // tokens one score workgroup walks
constexpr int kTopkThreads = 1024;

__device__ __forceinline__ void lds_dma16(const void *gsrc, void *ldst) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)gsrc,
                                   (__attribute__((address_space(3))) void *)ldst, 16, 0, 0);
}

__device__ __forceinline__ void lds_dma4(const void *gsrc, void *ldst) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)gsrc,
                                   (__attribute__((address_space(3))) void *)ldst, 4, 0, 0);
}

// e4m3fn code -> x = value * 2^9 (integer), NaN codes -> 0.
__device__ __forceinline__ int e4m3_x(uint32_t c) {
  const int e = (c >> 3) & 15, m = c & 7;
  int x = (e == 0) ? m : ((8 + m) << (e - 1));
  if (e == 15 && m == 7) x = 0;
  return (c & 0x80) ? -x : x;
}

// Signed 7-bit piece `pc` of x (sign-magnitude split), as a byte.
__device__ __forceinline__ uint32_t piece_byte(int x, int pc) {
  const int mag = x < 0 ? -x : x;
  const int v = (mag >> (7 * pc)) & 127;
  return (uint32_t)(x < 0 ? -v : v) & 0xffu;
}

__device__ __forceinline__ int piece_level(int x) {
  const int mag = x < 0 ? -x : x;
  return mag >= (1 << 14) ? 2 : (mag >= (1 << 7) ? 1 : 0);
}

// ---- q pieces ------------------------------------------------------------

__global__ __launch_bounds__(256) void dsa_idx_prep_q_kernel(IndexerParams p) {
  __shared__ int s_level;
  const int t = blockIdx.x;
  if (threadIdx.x == 0) s_level = 0;
  __syncthreads();
  int level = 0;
  const int chunks = p.Hi * (kIdxDim / 16);
  for (int c = threadIdx.x; c < chunks; c += 256) {
    const int h = c / (kIdxDim / 16), part = c % (kIdxDim / 16);
    const uint4 raw = *(const uint4 *)(p.q + ((int64_t)t * p.Hi + h) * kIdxDim + part * 16);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
    uint4 out[3];
    uint32_t *o[3] = {&out[0].x, &out[1].x, &out[2].x};
#pragma unroll
    for (int pc = 0; pc < 3; ++pc)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t packed = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) packed |= piece_byte(e4m3_x((w[i] >> (8 * b)) & 0xff), pc) << (8 * b);
        o[pc][i] = packed;
      }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int b = 0; b < 4; ++b) level = max(level, piece_level(e4m3_x((w[i] >> (8 * b)) & 0xff)));
    int8_t *dst = p.q_pieces + (((int64_t)t * p.Hi + h) * 3) * kIdxDim + part * 16;
#pragma unroll
    for (int pc = 0; pc < 3; ++pc) *(uint4 *)(dst + pc * kIdxDim) = out[pc];
  }
  atomicMax(&s_level, level);
  __syncthreads();
  if (threadIdx.x == 0) p.q_flags[t] = s_level;
}

// ---- scores --------------------------------------------------------------

template <int NP>
__device__ __forceinline__ void pair_products(const i32x4 (&aq)[2][3], const i32x4 (&kb)[2][3],
                                              i32x4 (&P)[3][3]) {
#pragma unroll
  for (int a = 0; a < NP; ++a)
#pragma unroll
    for (int b = 0; b < NP; ++b) {
      i32x4 c = {0, 0, 0, 0};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) c = __builtin_amdgcn_mfma_i32_16x16x64_i8(aq[ks][a], kb[ks][b], c, 0, 0, 0);
      P[a][b] = c;
    }
}

__global__ __launch_bounds__(256, 1) void dsa_idx_score_kernel(IndexerParams p) {
  // The score's rounding order is part of its definition: no fused
  // multiply-adds.  The pragma covers only the operators written in this
  // body (library helpers such as __fmul_rn are compiled under the global
  // contraction setting and would fuse after inlining), so the products and
  // sums below are plain operators.
#pragma clang fp contract(off)
  // double-buffered q pieces of one token [64 heads max][3][128] + its weights
  constexpr int kQBytes = 64 * 3 * kIdxDim;
  __shared__ __attribute__((aligned(16))) int8_t lds_q[2][kQBytes];
  __shared__ __attribute__((aligned(16))) float lds_w[2][64];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r16 = lane & 15, g = lane >> 4;
  const int pos0 = blockIdx.x * kScoreSlots + wave * (kSlotBlocks * 16);
  const int t_begin = blockIdx.y * kTokensPerGroup;
  const int t_end = min(p.T, t_begin + kTokensPerGroup);

  // ---- this lane's k pieces (B operands) and scales, decoded once
  i32x4 kb[kSlotBlocks][2][3];
  float kscale[kSlotBlocks];
  int klevel = 0;
#pragma unroll
  for (int sb = 0; sb < kSlotBlocks; ++sb) {
    const int s = pos0 + sb * 16 + r16;
    const bool ok = s < p.S;
    kscale[sb] = ok ? p.k_scale[s] * 0x1p-18f : 0.f;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      uint4 raw = make_uint4(0, 0, 0, 0);
      if (ok) raw = *(const uint4 *)(p.k + (int64_t)s * kIdxDim + ks * 64 + g * 16);
      const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
      for (int pc = 0; pc < 3; ++pc)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          uint32_t packed = 0;
#pragma unroll
          for (int b = 0; b < 4; ++b) packed |= piece_byte(e4m3_x((w[i] >> (8 * b)) & 0xff), pc) << (8 * b);
          kb[sb][ks][pc][i] = (int)packed;
        }
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int b = 0; b < 4; ++b) klevel = max(klevel, piece_level(e4m3_x((w[i] >> (8 * b)) & 0xff)));
    }
  }
  // wave-uniform level of this wave's positions
  klevel = __ballot(klevel == 2) ? 2 : (__ballot(klevel == 1) ? 1 : 0);

  // ---- stage each token's q pieces (contiguous [Hi][3][128] bytes) and its
  // head weights into LDS with global_load_lds (1 KB per instruction, split
  // over the waves); the next token streams in while the current one is
  // computed.
  const int n_kb = p.Hi * 3 * kIdxDim / 1024;  // 1 KB DMA instructions per token
  auto stage_token = [&](int tt, int bf) {
    const int8_t *src = p.q_pieces + (int64_t)tt * p.Hi * 3 * kIdxDim;
    for (int j = wave; j < n_kb; j += 4)
      lds_dma16(src + j * 1024 + lane * 16, &lds_q[bf][j * 1024]);
    if (wave == 0 && lane < p.Hi) lds_dma4(p.w + (int64_t)tt * p.Hi + lane, &lds_w[bf][0]);
  };
  if (t_begin < t_end) stage_token(t_begin, 0);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  for (int t = t_begin; t < t_end; ++t) {
    const int buf = (t - t_begin) & 1;
    if (t + 1 < t_end) stage_token(t + 1, buf ^ 1);
    const int qlevel = p.q_flags[t];
    const int level = max(qlevel, klevel);  // wave-uniform
    const int8_t *qt = lds_q[buf];
    const float *wt = lds_w[buf];

    float z[4][kSlotBlocks];  // per head block: (G0 + G1) + (G2 + G3)
#pragma unroll
    for (int hb = 0; hb < 4; ++hb) {
      if (hb * 16 >= p.Hi) break;  // wave-uniform
      i32x4 aq[2][3];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int pc = 0; pc < 3; ++pc)
          aq[ks][pc] = *(const i32x4 *)(qt + ((hb * 16 + r16) * 3 + pc) * kIdxDim + ks * 64 + g * 16);
      const float4 wv = *(const float4 *)(wt + hb * 16 + 4 * g);
      const float wh[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
      for (int sb = 0; sb < kSlotBlocks; ++sb) {
        i32x4 P[3][3];
        float f[4];
        if (level <= 1) {
          pair_products<2>(aq, kb[sb], P);
          bool small = true;
#pragma unroll
          for (int i = 0; i < 4; ++i) small &= (P[1][1][i] < (1 << 16)) && (P[1][1][i] > -(1 << 16));
          if (__ballot(!small) == 0) {
            // |D| < 2^31: exact in int32, one RNE conversion
#pragma unroll
            for (int i = 0; i < 4; ++i)
              f[i] = (float)(P[0][0][i] + (P[0][1][i] + P[1][0][i]) * 128 + P[1][1][i] * 16384);
          } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const double D = (double)P[0][0][i] + 128.0 * (double)(P[0][1][i] + P[1][0][i]) +
                               16384.0 * (double)P[1][1][i];
              f[i] = (float)D;
            }
          }
        } else {
          pair_products<3>(aq, kb[sb], P);
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            double D = 0.0;
#pragma unroll
            for (int a = 0; a < 3; ++a)
#pragma unroll
              for (int b = 0; b < 3; ++b) D += (double)P[a][b][i] * (double)(1 << (7 * (a + b)));
            f[i] = (float)D;
          }
        }
        // a = fl32(d32 * scale) (2^-18 folded into the scale); r = max(a, 0);
        // v = fl32(w * r); G over this lane's 4 heads in order
        float G = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float a = f[i] * kscale[sb];
          const float r = a > 0.f ? a : 0.f;
          const float v = wh[i] * r;
          G = (i == 0) ? v : G + v;
        }
        const float y = G + __shfl_xor(G, 16);
        z[hb][sb] = y + __shfl_xor(y, 32);
      }
    }
    float acc[kSlotBlocks];
#pragma unroll
    for (int sb = 0; sb < kSlotBlocks; ++sb) {
      float a = 0.f;
#pragma unroll
      for (int hb = 0; hb < 4; ++hb)
        if (hb * 16 < p.Hi) a = a + z[hb][sb];
      acc[sb] = a;
    }
    if (g == 0) {
#pragma unroll
      for (int sb = 0; sb < kSlotBlocks; ++sb) {
        const int s = pos0 + sb * 16 + r16;
        if (s < p.S) p.scores[(int64_t)t * p.S + s] = (s > p.limit[t]) ? -INFINITY : acc[sb];
      }
    }
    // token t+1 landed, and every wave is done with buffer buf before the
    // next iteration refills it
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
  }
}

// ---- top-k ---------------------------------------------------------------

__device__ __forceinline__ uint32_t order_key(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f == 0.f ? 0.f : f);  // -0 -> +0
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Exclusive prefix sum over the 1024 threads of the block; returns the
// exclusive sum and writes the total to *total.
__device__ int block_exclusive_scan(int v, int *scratch, int *total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) scratch[wave] = x;
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int w = 0; w < kTopkThreads / 64; ++w) {
      const int c = scratch[w];
      scratch[w] = run;
      run += c;
    }
    scratch[kTopkThreads / 64] = run;
  }
  __syncthreads();
  const int ex = scratch[wave] + x - v;
  *total = scratch[kTopkThreads / 64];
  __syncthreads();
  return ex;
}

__global__ __launch_bounds__(kTopkThreads) void dsa_idx_topk_kernel(IndexerParams p) {
  __shared__ uint32_t hist[256];
  __shared__ int scan_scratch[kTopkThreads / 64 + 1];
  __shared__ uint32_t s_prefix, s_mask;
  __shared__ int s_need;

  const int t = blockIdx.x;
  const float *row = p.scores + (int64_t)t * p.S;
  int32_t *out = p.out + (int64_t)t * p.topk;
  const int n = max(0, min(p.S, p.limit[t] + 1));  // candidates 0..n-1
  const int K = p.topk;

  auto emit = [&](int slot_pos, int rank) {
    int v = slot_pos;
    if (p.block_table != nullptr) {
      const int32_t page = p.block_table[(int64_t)t * p.bt_stride + slot_pos / p.page_size];
      v = page * p.page_size + slot_pos % p.page_size;
    }
    out[rank] = v;
  };

  if (n <= K) {
    for (int i = threadIdx.x; i < K; i += kTopkThreads) {
      if (i < n) emit(i, i);
      else out[i] = -1;
    }
    return;
  }

  // ---- radix select of the K-th largest key
  if (threadIdx.x == 0) {
    s_prefix = 0;
    s_mask = 0;
    s_need = K;
  }
  for (int shift = 24; shift >= 0; shift -= 8) {
    if (threadIdx.x < 256) hist[threadIdx.x] = 0;
    __syncthreads();
    const uint32_t prefix = s_prefix, mask = s_mask;
    for (int i = threadIdx.x; i < n; i += kTopkThreads) {
      const uint32_t key = order_key(row[i]);
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (threadIdx.x < 64) {
      // lane l owns bins 4l..4l+3; suffix sums from the top bin down
      const int l = threadIdx.x;
      const uint32_t c0 = hist[4 * l], c1 = hist[4 * l + 1], c2 = hist[4 * l + 2], c3 = hist[4 * l + 3];
      const uint32_t local = c0 + c1 + c2 + c3;
      uint32_t above = 0;  // total of lanes > l
      uint32_t x = local;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_down(x, o);
        if (l + o < 64) x += y;
      }
      above = x - local;
      const int need = s_need;
      // bins within this lane, from 4l+3 down
      uint32_t cum = above;
      const uint32_t cs[4] = {c0, c1, c2, c3};
#pragma unroll
      for (int b = 3; b >= 0; --b) {
        if ((int)cum < need && (int)(cum + cs[b]) >= need) {
          s_prefix = prefix | ((uint32_t)(4 * l + b) << shift);
          s_mask = mask | (255u << shift);
          s_need = need - (int)cum;
        }
        cum += cs[b];
      }
    }
    __syncthreads();
  }
  const uint32_t tau = s_prefix;
  const int need_eq = s_need;  // ties at tau to take, lowest positions first

  // ---- ordered compaction: thread i owns positions [i*chunk, (i+1)*chunk)
  const int chunk = (n + kTopkThreads - 1) / kTopkThreads;
  const int b0 = min(n, threadIdx.x * chunk), b1 = min(n, b0 + chunk);
  int n_gt = 0, n_eq = 0;
  for (int i = b0; i < b1; ++i) {
    const uint32_t key = order_key(row[i]);
    n_gt += key > tau;
    n_eq += key == tau;
  }
  int tot;
  const int eq_base = block_exclusive_scan(n_eq, scan_scratch, &tot);
  const int take_eq = max(0, min(n_eq, need_eq - eq_base));
  const int out_base = block_exclusive_scan(n_gt + take_eq, scan_scratch, &tot);
  int o = out_base, eq_seen = 0;
  for (int i = b0; i < b1; ++i) {
    const uint32_t key = order_key(row[i]);
    bool sel = key > tau;
    if (key == tau) {
      sel = eq_seen < take_eq;
      ++eq_seen;
    }
    if (sel) emit(i, o++);
  }
  for (int i = tot + threadIdx.x; i < K; i += kTopkThreads) out[i] = -1;
}

}  // namespace

hipError_t launch_indexer(const IndexerParams &p, hipStream_t stream) {
  if (p.T == 0) return hipSuccess;
  hipLaunchKernelGGL(dsa_idx_prep_q_kernel, dim3(p.T), dim3(256), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (p.S > 0) {
    const dim3 grid((p.S + kScoreSlots - 1) / kScoreSlots,
                    (p.T + kTokensPerGroup - 1) / kTokensPerGroup);
    hipLaunchKernelGGL(dsa_idx_score_kernel, grid, dim3(256), 0, stream, p);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (p.topk > 0) {
    hipLaunchKernelGGL(dsa_idx_topk_kernel, dim3(p.T), dim3(kTopkThreads), 0, stream, p);
    e = hipGetLastError();
  }
  return e;
}

}  // namespace dsa

