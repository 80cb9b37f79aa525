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
// Work decomposition.  One workgroup = one (token, top-k chunk, 16-head
// group) with four independent waves.  Each wave walks its own 32-key tiles
// of the chunk: it gathers the 32 selected rows (1024 B ckv + 128 B kpe each)
// with global_load_lds_dwordx4 straight into a private LDS tile (no VGPR
// staging, 36 row loads in flight per wave), then
//   S^T[32 keys x 16 heads] = K[keys x 576] . Q^T          (bf16 MFMA 16x16x32)
//   online softmax in fp32 (log2 domain)
//   O^T[512 x 16 heads]    += V^T[512 x 32 keys] . P^T      (bf16 MFMA 16x16x32)
// Computing S^T (keys as the MFMA M dimension) leaves P^T in exactly the
// lane layout the PV product takes as its B operand, so P never round-trips
// through LDS.  At the end the four waves' (m, l, O) states are merged in LDS
// and the workgroup writes either the final bf16 output and lse (one chunk per
// token) or an unnormalised fp32 partial that dsa_attn_combine merges with
// log-sum-exp weights (reference merge algebra: kernel.py:461-493).
//
// MFMA 16x16x32 bf16 lane layout used throughout (lane = 16*g + r):
//   A (16 x 32): lane holds row r, k-slots 8g..8g+7
//   B (32 x 16): lane holds column r, k-slots 8g..8g+7
//   D (16 x 16): lane holds column r, rows 4g..4g+3
// Only the A/B k-slot assignment being identical matters for a product, so
// the kernel assigns k-slots to features or keys as convenient.
#include "dsa_internal.h"

namespace dsa {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));

// LDS tile geometry (bytes).  A ckv row is padded from 1024 to 1040 B so the
// 16 rows one MFMA operand read touches fall in distinct banks; kpe rows are
// gathered 8 per DMA instruction in chunk-major order (lane i of the DMA
// holds 16-byte chunk i/8 of row i%8), so a column read of 16 rows hits 16
// consecutive chunks.
constexpr int kCkvPitch = 1024 + 16;
constexpr int kKpeGroupPitch = 1024 + 128;
constexpr int kCkvTileBytes = kKeysPerTile * kCkvPitch;
constexpr int kKpeTileBytes = (kKeysPerTile / 8) * kKpeGroupPitch;
constexpr int kWaveTileBytes = kCkvTileBytes + kKpeTileBytes;
constexpr int kLdsBytes = kAttnWaves * kWaveTileBytes;
constexpr int kMergeBytes = kAttnWaves * 32 * 64 * 16;
static_assert(kMergeBytes <= kLdsBytes, "merge buffer must fit in the tile buffers");
static_assert(kLdsBytes + 2 * kAttnWaves * 16 * 4 <= 160 * 1024, "LDS budget of one gfx950 CU");

__device__ __forceinline__ void lds_dma16(const void *gsrc, void *ldst) {
  __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)gsrc,
                                   (__attribute__((address_space(3))) void *)ldst, 16, 0, 0);
}

__device__ __forceinline__ int64_t readlane64(int64_t v, int lane) {
  const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, lane);
  const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)((uint64_t)v >> 32), lane);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ unsigned short f32_to_bf16_rne(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (unsigned short)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (unsigned short)(u >> 16);
}

__global__ __launch_bounds__(kAttnWaves * 64, 1) void dsa_attn_partial_kernel(AttnParams p) {
  __shared__ __attribute__((aligned(16))) char lds[kLdsBytes];
  __shared__ float lds_m[kAttnWaves][16];
  __shared__ float lds_l[kAttnWaves][16];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int t = blockIdx.x / p.num_splits;
  const int split = blockIdx.x - t * p.num_splits;
  const int r16 = lane & 15;
  const int g = lane >> 4;
  const int head = blockIdx.y * kHeadsPerGroup + r16;

  const int k_begin = split * p.chunk;
  const int k_end = min(p.K, k_begin + p.chunk);
  const int n_keys = max(0, k_end - k_begin);
  const int n_tiles = (n_keys + kKeysPerTile - 1) / kKeysPerTile;

  // Q^T as the B operand of S^T = K Q^T: k-step s covers features 32s..32s+31
  // (s < 16: q_nope; s = 16, 17: q_pe), this lane holds 8g..8g+7 of them.
  bf16x8 qreg[18];
  {
    const char *qn = p.q_nope + t * p.qn_st + head * p.qn_sh + g * 16;
#pragma unroll
    for (int s = 0; s < 16; ++s) qreg[s] = *(const bf16x8 *)(qn + s * 64);
    const char *qp = p.q_pe + t * p.qp_st + head * p.qp_sh + g * 16;
#pragma unroll
    for (int s = 0; s < 2; ++s) qreg[16 + s] = *(const bf16x8 *)(qp + s * 64);
  }

  f32x4 acc[32];
#pragma unroll
  for (int i = 0; i < 32; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY;  // running max of x*log2(e), this lane's head
  float l_run = 0.f;        // running sum over this lane's keys (reduced at the end)

  char *tile_ckv = lds + wave * kWaveTileBytes;
  char *tile_kpe = tile_ckv + kCkvTileBytes;
  const int32_t *idx_row = p.idx + (int64_t)t * p.idx_st;

  for (int tile = wave; tile < n_tiles; tile += kAttnWaves) {
    const int kb = k_begin + tile * kKeysPerTile;
    const int nk = min(kKeysPerTile, k_end - kb);

    // ---- slot ids of this tile's keys (lane & 31) and their row offsets
    int slot = -1;
    if ((lane & 31) < nk) slot = idx_row[kb + (lane & 31)];
    const bool valid = slot >= 0 && (int64_t)slot < p.num_slots;
    const uint32_t vmask = (uint32_t)__ballot(valid);
    int64_t ckv_off = 0, kpe_off = 0;
    if (valid) {
      const uint32_t pg = (uint32_t)slot / (uint32_t)p.page_size;
      const uint32_t of = (uint32_t)slot - pg * (uint32_t)p.page_size;
      ckv_off = (int64_t)pg * p.ckv_sp + (int64_t)of * p.ckv_so;
      kpe_off = (int64_t)pg * p.kpe_sp + (int64_t)of * p.kpe_so;
    }

    // ---- gather: 32 ckv rows (one 1 KB DMA each) + 4 x 8 kpe rows.
    // Invalid or missing keys get a zero row so padding never feeds NaN/Inf
    // garbage into the MFMAs (their probabilities are exactly zero).
#pragma unroll
    for (int r = 0; r < kKeysPerTile; ++r) {
      char *dst = tile_ckv + r * kCkvPitch;
      if ((vmask >> r) & 1u) {
        lds_dma16(p.ckv + readlane64(ckv_off, r) + lane * 16, dst);
      } else {
        *(uint4 *)(dst + lane * 16) = make_uint4(0u, 0u, 0u, 0u);
      }
    }
#pragma unroll
    for (int q = 0; q < kKeysPerTile / 8; ++q) {
      const int r = q * 8 + (lane & 7);
      const int64_t off = __shfl(kpe_off, r);
      char *dst = tile_kpe + q * kKpeGroupPitch;
      if ((vmask >> r) & 1u) {
        lds_dma16(p.kpe + off + (lane >> 3) * 16, dst);
      } else {
        *(uint4 *)(dst + lane * 16) = make_uint4(0u, 0u, 0u, 0u);
      }
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");

    // ---- S^T = K . Q^T for two 16-key blocks
    f32x4 sacc[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      f32x4 c = {0.f, 0.f, 0.f, 0.f};
      const char *rowp = tile_ckv + (b * 16 + r16) * kCkvPitch + g * 16;
#pragma unroll
      for (int s = 0; s < 16; ++s)
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const bf16x8 *)(rowp + s * 64), qreg[s], c,
                                                     0, 0, 0);
      const int kk = b * 16 + r16;
      const char *kp = tile_kpe + (kk >> 3) * kKpeGroupPitch + (kk & 7) * 16;
#pragma unroll
      for (int s = 0; s < 2; ++s)
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*(const bf16x8 *)(kp + (s * 4 + g) * 128),
                                                     qreg[16 + s], c, 0, 0, 0);
      sacc[b] = c;
    }

    // ---- online softmax (this lane: head r16, keys b*16 + 4g + i)
    float x[8];
    float mx = -INFINITY;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = b * 16 + 4 * g + i;
        const float v = ((vmask >> key) & 1u) ? sacc[b][i] * p.scale_log2 : -INFINITY;
        x[b * 4 + i] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const bool none = m_new == -INFINITY;
    const float alpha = none ? 1.f : fast_exp2(m_run - m_new);
    u16x8 pbits;
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float pv = none ? 0.f : fast_exp2(x[i] - m_new);
      psum += pv;
      pbits[i] = f32_to_bf16_rne(pv);
    }
    l_run = l_run * alpha + psum;
    m_run = m_new;
    const bf16x8 pB = __builtin_bit_cast(bf16x8, pbits);

    // ---- O^T += V^T . P^T: k-slot i of group g is key 4g+i (i<4) or 16+4g+(i-4)
    const char *vcol = tile_ckv + r16 * 2;
    const char *vrow[8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
      vrow[i] = vcol + ((i < 4) ? (4 * g + i) : (16 + 4 * g + i - 4)) * kCkvPitch;
#pragma unroll
    for (int fb = 0; fb < 32; ++fb) {
      u16x8 a;
#pragma unroll
      for (int i = 0; i < 8; ++i) a[i] = *(const unsigned short *)(vrow[i] + fb * 32);
      acc[fb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), pB,
                                                        acc[fb] * alpha, 0, 0, 0);
    }
  }

  // ---- merge the four waves' states through LDS
  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);
  __syncthreads();
  f32x4 *mbuf = (f32x4 *)lds;
#pragma unroll
  for (int fb = 0; fb < 32; ++fb) mbuf[(wave * 32 + fb) * 64 + lane] = acc[fb];
  if (lane < 16) {
    lds_m[wave][lane] = m_run;
    lds_l[wave][lane] = l_run;
  }
  __syncthreads();

  float mw[kAttnWaves];
  float M = -INFINITY;
#pragma unroll
  for (int w = 0; w < kAttnWaves; ++w) {
    mw[w] = lds_m[w][r16];
    M = fmaxf(M, mw[w]);
  }
  float aw[kAttnWaves];
  float L = 0.f;
#pragma unroll
  for (int w = 0; w < kAttnWaves; ++w) {
    aw[w] = (mw[w] == -INFINITY) ? 0.f : fast_exp2(mw[w] - M);
    L += aw[w] * lds_l[w][r16];
  }

  const bool final_out = p.num_splits == 1;
  const float inv = (M == -INFINITY) ? 0.f : 1.f / L;
#pragma unroll
  for (int j = 0; j < 32 / kAttnWaves; ++j) {
    const int fb = wave * (32 / kAttnWaves) + j;
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) o += aw[w] * mbuf[(w * 32 + fb) * 64 + lane];
    const int f0 = fb * 16 + 4 * g;
    if (final_out) {
      u16x4 ob;
#pragma unroll
      for (int i = 0; i < 4; ++i) ob[i] = f32_to_bf16_rne(o[i] * inv);
      *(u16x4 *)(p.out + t * p.out_st + head * p.out_sh + f0 * 2) = ob;
    } else {
      const int64_t row = ((int64_t)t * p.num_splits + split) * p.H + head;
      *(f32x4 *)(p.part_acc + row * kHeadDimCkv + f0) = o;
    }
  }
  if (wave == 0 && lane < 16) {
    if (final_out) {
      p.lse[t * p.lse_st + head * p.lse_sh] = (M == -INFINITY) ? -INFINITY : M + __log2f(L);
    } else {
      const int64_t row = ((int64_t)t * p.num_splits + split) * p.H + head;
      p.part_ml[row * 2 + 0] = M;
      p.part_ml[row * 2 + 1] = L;
    }
  }
}

// Log-sum-exp merge of the per-chunk partials (reference: dsa_reduce_kernel,
// kernel.py:437-493, with its -inf guards :475-476).  One workgroup per
// (token, head); 128 threads x 4 features.  Split order is fixed, so the
// result is deterministic.
__global__ __launch_bounds__(128) void dsa_attn_combine_kernel(AttnParams p) {
  const int t = blockIdx.x;
  const int head = blockIdx.y;
  const int S = p.num_splits;
  const int f0 = threadIdx.x * 4;
  const int64_t row0 = (int64_t)t * S * p.H + head;
  float M = -INFINITY;
  for (int s = 0; s < S; ++s) M = fmaxf(M, p.part_ml[(row0 + (int64_t)s * p.H) * 2]);
  float L = 0.f;
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < S; ++s) {
    const int64_t row = row0 + (int64_t)s * p.H;
    const float ms = p.part_ml[row * 2];
    const float a = (ms == -INFINITY) ? 0.f : fast_exp2(ms - M);
    L += a * p.part_ml[row * 2 + 1];
    o += a * *(const f32x4 *)(p.part_acc + row * kHeadDimCkv + f0);
  }
  const float inv = (M == -INFINITY) ? 0.f : 1.f / L;
  u16x4 ob;
#pragma unroll
  for (int i = 0; i < 4; ++i) ob[i] = f32_to_bf16_rne(o[i] * inv);
  *(u16x4 *)(p.out + t * p.out_st + head * p.out_sh + f0 * 2) = ob;
  if (threadIdx.x == 0)
    p.lse[t * p.lse_st + head * p.lse_sh] = (M == -INFINITY) ? -INFINITY : M + __log2f(L);
}

}  // namespace

hipError_t launch_attention(const AttnParams &p, hipStream_t stream) {
  if (p.T == 0) return hipSuccess;
  const dim3 grid(p.T * p.num_splits, p.H / kHeadsPerGroup);
  hipLaunchKernelGGL(dsa_attn_partial_kernel, grid, dim3(kAttnWaves * 64), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || p.num_splits == 1) return e;
  hipLaunchKernelGGL(dsa_attn_combine_kernel, dim3(p.T, p.H), dim3(128), 0, stream, p);
  return hipGetLastError();
}

}  // namespace dsa
