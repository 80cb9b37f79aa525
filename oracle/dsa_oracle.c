/*
 * dsa_oracle.c -- CPU restatement of the reference's DeepSeek sparse attention
 * (DSA) path.  TEST INFRASTRUCTURE ONLY: this file is the checker that the HIP
 * kernels are compared against.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product library never does.
 *
 * Functions and the reference code each one restates:
 *
 *   oracle_dsa_attention   solution/triton/indexer_kernel.py:436-497 (run()):
 *                          per token, drop -1 entries (:470-471), an empty row
 *                          gives zeros and lse=-inf (:473-475), gather by flat
 *                          slot id (:458-459,477-481), logits=(qn.Kc^T+qp.Kp^T)
 *                          *sm_scale (:486-487), lse=logsumexp/ln2 (:490),
 *                          out=bf16(softmax.Kc) (:493-495).  The reference's
 *                          constant asserts (:444-448) are not restated: any
 *                          H, page size and top-k are accepted.  Arithmetic is
 *                          fp64 (the reference uses fp32 from bf16-exact
 *                          inputs; the difference is ~1e-7 relative).
 *
 *   oracle_e4m3_decode     OCP float8 e4m3fn decode (sign, 4-bit exponent with
 *                          bias 7, 3-bit mantissa, subnormals, 0x7f/0xff NaN).
 *
 *   oracle_indexer_scores  the lightning-indexer score, whose structure follows
 *                          indexer_kernel.py:185-275 (dequantize -> dot -> ReLU
 *                          -> head weight -> sum over heads), in the factored
 *                          form scale[s] * sum_h w[t,h]*relu(dot) (equal to
 *                          sum_h w*relu(dot*scale) for a positive scale), with
 *                          one exact rounding order:
 *                            D   = 2^18 * sum_j q[t,h,j]*k[s,j]  (exact: fp8
 *                                  products are exact and the 128-term sum
 *                                  spans < 53 bits, so fp64 accumulation is
 *                                  exact)
 *                            r_h = fl32(max(D, 0))
 *                            the heads form 4 groups of Hi/4 consecutive
 *                            heads; G_g = fma(w[t,h], r_h, G_g) over group g's
 *                            heads in ascending order, from G_g = 0
 *                            total = fl32(fl32(G_0 + G_1) + fl32(G_2 + G_3))
 *                            score = fl32(total * c_s),
 *                                    c_s = fl32(scale[s] * 2^-18)
 *                          (The reference's head sum, a Triton tl.sum, has no
 *                          defined order; this one is fixed so that the GPU
 *                          reproduces it bit for bit.)  Positions s > limit[t]
 *                          are masked (-inf).  Hi must be a multiple of 16.
 *
 *   oracle_topk            top-k per row by (score desc, index asc), which is
 *                          what indexer_kernel.py:289-343 intends (strict '>'
 *                          keeps the earlier index on ties, :333).  Masked
 *                          positions are never selected; rows with fewer than
 *                          k candidates are padded with -1.
 *
 * Build: oracle/build_oracle.sh (gcc -O2 -ffp-contract=off -fopenmp).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define ORACLE_OK 0
#define ORACLE_EINVAL 1
#define ORACLE_ENOMEM 2

static inline float bf16_to_f32(uint16_t b) {
  uint32_t u = ((uint32_t)b) << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* fp32 -> bf16, round to nearest even; NaN stays NaN (quiet). */
static inline uint16_t f32_to_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

uint16_t oracle_f32_to_bf16(float f) { return f32_to_bf16(f); }

/*
 * q_nope [T,H,Dc], q_pe [T,H,Dp], ckv [slots,Dc], kpe [slots,Dp] (bf16 bits,
 * contiguous; a paged cache [pages,ps,D] is the same memory viewed flat),
 * idx [T,K] int32 slot ids (-1 = pad).  Writes out [T,H,Dc] bf16 bits and
 * lse [T,H] (base 2).  Returns ORACLE_EINVAL if an id is neither -1 nor in
 * [0, slots) -- the reference's tensor indexing would raise there.
 * nthreads <= 0 means the OpenMP default.
 */
int oracle_dsa_attention(const uint16_t *q_nope, const uint16_t *q_pe,
                         const uint16_t *ckv, const uint16_t *kpe,
                         const int32_t *idx, int64_t T, int64_t H, int64_t K,
                         int64_t Dc, int64_t Dp, int64_t slots, float sm_scale,
                         uint16_t *out, float *lse, int nthreads) {
  if (T < 0 || H <= 0 || K < 0 || Dc <= 0 || Dp < 0 || slots < 0) return ORACLE_EINVAL;
  for (int64_t i = 0; i < T * K; ++i)
    if (idx[i] != -1 && (idx[i] < 0 || idx[i] >= slots)) return ORACLE_EINVAL;
  int status = ORACLE_OK;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#else
  (void)nthreads;
#endif
#pragma omp parallel
  {
    double *logit = (double *)malloc(sizeof(double) * (size_t)(K > 0 ? K : 1) * (size_t)H);
    double *qn = (double *)malloc(sizeof(double) * (size_t)(H * Dc));
    double *qp = (double *)malloc(sizeof(double) * (size_t)(H * (Dp > 0 ? Dp : 1)));
    double *row = (double *)malloc(sizeof(double) * (size_t)(Dc + Dp));
    double *acc = (double *)malloc(sizeof(double) * (size_t)(H * Dc));
    double *mx = (double *)malloc(sizeof(double) * (size_t)H);
    double *sum = (double *)malloc(sizeof(double) * (size_t)H);
    int64_t *sel = (int64_t *)malloc(sizeof(int64_t) * (size_t)(K > 0 ? K : 1));
    if (!logit || !qn || !qp || !row || !acc || !mx || !sum || !sel) {
#pragma omp atomic write
      status = ORACLE_ENOMEM;
    } else {
#pragma omp for schedule(dynamic, 1)
      for (int64_t t = 0; t < T; ++t) {
        /* valid_mask = indices != -1; valid_indices = indices[valid_mask] (:470-471) */
        int64_t n = 0;
        for (int64_t j = 0; j < K; ++j)
          if (idx[t * K + j] != -1) sel[n++] = idx[t * K + j];
        if (n == 0) { /* empty row: output zeros, lse stays -inf (:473-475) */
          for (int64_t h = 0; h < H; ++h) {
            memset(out + (t * H + h) * Dc, 0, sizeof(uint16_t) * (size_t)Dc);
            lse[t * H + h] = -INFINITY;
          }
          continue;
        }
        for (int64_t h = 0; h < H; ++h) {
          for (int64_t d = 0; d < Dc; ++d) qn[h * Dc + d] = bf16_to_f32(q_nope[(t * H + h) * Dc + d]);
          for (int64_t d = 0; d < Dp; ++d) qp[h * Dp + d] = bf16_to_f32(q_pe[(t * H + h) * Dp + d]);
        }
        /* logits = (qn @ Kc.T + qp @ Kp.T) * sm_scale (:486-487) */
        for (int64_t j = 0; j < n; ++j) {
          for (int64_t d = 0; d < Dc; ++d) row[d] = bf16_to_f32(ckv[sel[j] * Dc + d]);
          for (int64_t d = 0; d < Dp; ++d) row[Dc + d] = bf16_to_f32(kpe[sel[j] * Dp + d]);
          for (int64_t h = 0; h < H; ++h) {
            double s = 0.0;
            for (int64_t d = 0; d < Dc; ++d) s += qn[h * Dc + d] * row[d];
            for (int64_t d = 0; d < Dp; ++d) s += qp[h * Dp + d] * row[Dc + d];
            logit[h * n + j] = s * (double)sm_scale;
          }
        }
        /* lse = logsumexp(logits) / ln 2 (:490) */
        for (int64_t h = 0; h < H; ++h) {
          const double *x = logit + h * n;
          double m = -INFINITY;
          for (int64_t j = 0; j < n; ++j) m = x[j] > m ? x[j] : m;
          double sm = 0.0;
          for (int64_t j = 0; j < n; ++j) sm += exp(x[j] - m);
          mx[h] = m;
          sum[h] = sm;
          lse[t * H + h] = (float)((m + log(sm)) / log(2.0));
        }
        /* out = softmax(logits) @ Kc, cast to bf16 (:493-495) */
        for (int64_t i = 0; i < H * Dc; ++i) acc[i] = 0.0;
        for (int64_t j = 0; j < n; ++j) {
          for (int64_t d = 0; d < Dc; ++d) row[d] = bf16_to_f32(ckv[sel[j] * Dc + d]);
          for (int64_t h = 0; h < H; ++h) {
            const double p = exp(logit[h * n + j] - mx[h]) / sum[h];
            double *a = acc + h * Dc;
            for (int64_t d = 0; d < Dc; ++d) a[d] += p * row[d];
          }
        }
        for (int64_t i = 0; i < H * Dc; ++i) out[t * H * Dc + i] = f32_to_bf16((float)acc[i]);
      }
    }
    free(logit);
    free(qn);
    free(qp);
    free(row);
    free(acc);
    free(mx);
    free(sum);
    free(sel);
  }
  return status;
}

/* OCP e4m3fn: value = (-1)^s * 2^(E-7) * (1 + m/8) for E > 0, 2^-6 * m/8 for
 * E == 0; E == 15 && m == 7 is NaN (no infinities). */
float oracle_e4m3_decode(uint8_t b) {
  int s = b >> 7, E = (b >> 3) & 0xf, m = b & 7;
  float v;
  if (E == 15 && m == 7) return NAN;
  if (E == 0)
    v = ldexpf((float)m, -9);
  else
    v = ldexpf((float)(8 + m), E - 10);
  return s ? -v : v;
}

/*
 * q [T,Hi,D] e4m3 bytes, k [S,D] e4m3 bytes, kscale [S] fp32, w [T,Hi] fp32,
 * limit [T] int64 (position s is a candidate iff s <= limit[t]).
 * scores [T,S] fp32; masked positions get -inf.
 */
int oracle_indexer_scores(const uint8_t *q, const uint8_t *k, const float *kscale,
                          const float *w, const int64_t *limit, int64_t T, int64_t Hi,
                          int64_t D, int64_t S, float *scores, int nthreads) {
  if (T < 0 || Hi <= 0 || Hi % 16 != 0 || D <= 0 || S < 0) return ORACLE_EINVAL;
  float lut[256];
  for (int i = 0; i < 256; ++i) lut[i] = oracle_e4m3_decode((uint8_t)i);
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#else
  (void)nthreads;
#endif
#pragma omp parallel for schedule(static)
  for (int64_t t = 0; t < T; ++t) {
    for (int64_t s = 0; s < S; ++s) {
      if (s > limit[t]) {
        scores[t * S + s] = -INFINITY;
        continue;
      }
      const int64_t quarter = Hi / 4;
      const uint8_t *ks = k + s * D;
      float G[4];
      for (int g = 0; g < 4; ++g) {
        float acc = 0.0f;
        for (int64_t h = g * quarter; h < (g + 1) * quarter; ++h) {
          const uint8_t *qh = q + (t * Hi + h) * D;
          double d = 0.0;
          for (int64_t j = 0; j < D; ++j) d += (double)lut[qh[j]] * (double)lut[ks[j]];
          const double dscaled = d * 262144.0; /* exact: a power of two */
          const float r = (float)(dscaled > 0.0 ? dscaled : 0.0);
          acc = fmaf(w[t * Hi + h], r, acc);
        }
        G[g] = acc;
      }
      volatile float g01 = G[0] + G[1];
      volatile float g23 = G[2] + G[3];
      volatile float total = g01 + g23;
      volatile float cs = kscale[s] * 0x1p-18f;
      scores[t * S + s] = total * cs;
    }
  }
  return ORACLE_OK;
}

typedef struct {
  float score;
  int32_t pos;
} cand_t;

static int cand_cmp(const void *a, const void *b) {
  const cand_t *x = (const cand_t *)a, *y = (const cand_t *)b;
  if (x->score > y->score) return -1;
  if (x->score < y->score) return 1;
  return (x->pos > y->pos) - (x->pos < y->pos);
}

/* out [T,k] int32 in rank order (score desc, position asc), -1 padded. */
int oracle_topk(const float *scores, const int64_t *limit, int64_t T, int64_t S, int64_t kk,
                int32_t *out) {
  if (T < 0 || S < 0 || kk < 0 || S > 0x7fffffff) return ORACLE_EINVAL;
  cand_t *c = (cand_t *)malloc(sizeof(cand_t) * (size_t)(S > 0 ? S : 1));
  if (!c) return ORACLE_ENOMEM;
  for (int64_t t = 0; t < T; ++t) {
    int64_t n = 0;
    for (int64_t s = 0; s < S && s <= limit[t]; ++s) {
      c[n].score = scores[t * S + s];
      c[n].pos = (int32_t)s;
      ++n;
    }
    qsort(c, (size_t)n, sizeof(cand_t), cand_cmp);
    for (int64_t j = 0; j < kk; ++j) out[t * kk + j] = j < n ? c[j].pos : -1;
  }
  free(c);
  return ORACLE_OK;
}
