/*
 * CPU oracle for the tensor-op path: TEST INFRASTRUCTURE ONLY (the checker,
 * never the product). See oracle.h for the restated reference loops.
 *
 * Loop-order note: every output element is accumulated in fp32 in exactly
 * the order the reference loop uses (bias/zero first, then the contraction
 * index ascending). Where the reference writes "for element { for i {...} }"
 * this file sometimes writes "for i { for element {...} }" with one
 * accumulator per element; each element still sees the same sequence of
 * separately rounded multiplies and adds (built with -ffp-contract=off), so
 * the result is bit-identical and the inner loop vectorises.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ numbers */

uint16_t oracle_f32_to_f16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  uint32_t sign = (u >> 16) & 0x8000u;
  uint32_t exp = (u >> 23) & 0xffu;
  uint32_t mant = u & 0x7fffffu;
  if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (mant ? (0x200u | (mant >> 13)) : 0u));
  int e = (int)exp - 127 + 15;
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign; /* below half the smallest subnormal */
    mant |= 0x800000u;
    int shift = 14 - e; /* f16 subnormal: value = m * 2^-24 */
    uint32_t m = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (m & 1u))) m++;
    return (uint16_t)(sign | m);
  }
  uint32_t r = sign | ((uint32_t)e << 10) | (mant >> 13);
  uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++; /* carry may roll into the exponent: correct */
  return (uint16_t)r;
}

float oracle_f16_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
  uint32_t mant = (uint32_t)h & 0x3ffu;
  uint32_t u;
  if (exp == 0) {
    float v = ldexpf((float)mant, -24);
    return sign ? -v : v;
  } else if (exp == 31) {
    u = sign | 0x7f800000u | (mant << 13);
  } else {
    u = sign | ((exp + 112u) << 23) | (mant << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

uint16_t oracle_f32_to_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x7fffffu)) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float oracle_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline float to_f32(int dtype, uint16_t v) {
  return dtype == ORACLE_BF16 ? oracle_bf16_to_f32(v) : oracle_f16_to_f32(v);
}

static inline uint16_t from_f32(int dtype, float v) {
  return dtype == ORACLE_BF16 ? oracle_f32_to_bf16(v) : oracle_f32_to_f16(v);
}

void oracle_to_f32(int dtype, const uint16_t *src, float *dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = to_f32(dtype, src[i]);
}

void oracle_from_f32(int dtype, const float *src, uint16_t *dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = from_f32(dtype, src[i]);
}

/* ------------------------------------------------------------------ inputs */

static inline uint64_t splitmix64(uint64_t *state) {
  uint64_t z = (*state += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

static inline double unit_double(uint64_t *state) { /* [0, 1) with 53 random bits */
  return (double)(splitmix64(state) >> 11) * (1.0 / 9007199254740992.0);
}

void oracle_fill_uniform(uint64_t seed, double lo, double hi, int dtype, uint16_t *out, size_t n) {
  uint64_t s = seed;
  for (size_t i = 0; i < n; ++i) out[i] = from_f32(dtype, (float)(lo + (hi - lo) * unit_double(&s)));
}

void oracle_fill_normal(uint64_t seed, double mean, double stddev, int dtype, uint16_t *out, size_t n) {
  /* Box-Muller in fp64, both outputs of each pair used (as Network.swift:115-129 does). */
  const double two_pi = 6.283185307179586476925286766559;
  uint64_t s = seed;
  for (size_t i = 0; i < n; i += 2) {
    double u1 = 1.0 - unit_double(&s); /* (0, 1] so log is finite */
    double u2 = unit_double(&s);
    double r = sqrt(-2.0 * log(u1));
    out[i] = from_f32(dtype, (float)(mean + stddev * r * cos(two_pi * u2)));
    if (i + 1 < n) out[i + 1] = from_f32(dtype, (float)(mean + stddev * r * sin(two_pi * u2)));
  }
}

static int pick_threads(int nthreads) {
#ifdef _OPENMP
  return nthreads > 0 ? nthreads : omp_get_max_threads();
#else
  (void)nthreads;
  return 1;
#endif
}

/* ------------------------------------------------------------------ GEMM */

void oracle_gemm(int dtype, int M, int N, int K, int trans_b, const uint16_t *A, const uint16_t *B,
                 const uint16_t *bias, float *C, int row_begin, int row_end, int nthreads) {
  /* matmul.swift:498-510: expected = Float(bias[n]); for i in 0..<K { expected += Float(A[i + m*K]) *
   * Float(B[i + n*K]) }. B is widened once into fp32 [K][N] so the n loop is contiguous. */
  if (row_begin < 0) row_begin = 0;
  if (row_end > M || row_end < 0) row_end = M;
  float *Bkn = (float *)malloc(sizeof(float) * (size_t)K * (size_t)N);
  float *biasf = (float *)malloc(sizeof(float) * (size_t)N);
  for (int i = 0; i < K; ++i)
    for (int n = 0; n < N; ++n)
      Bkn[(size_t)i * N + n] = to_f32(dtype, trans_b ? B[(size_t)n * K + i] : B[(size_t)i * N + n]);
  for (int n = 0; n < N; ++n) biasf[n] = bias ? to_f32(dtype, bias[n]) : 0.0f;
  int nt = pick_threads(nthreads);
#pragma omp parallel for schedule(static) num_threads(nt)
  for (int m = row_begin; m < row_end; ++m) {
    float *acc = C + (size_t)m * N;
    for (int n = 0; n < N; ++n) acc[n] = biasf[n];
    for (int i = 0; i < K; ++i) {
      const float a = to_f32(dtype, A[(size_t)m * K + i]);
      const float *brow = Bkn + (size_t)i * N;
      for (int n = 0; n < N; ++n) acc[n] += a * brow[n];
    }
  }
  free(Bkn);
  free(biasf);
}

/* ------------------------------------------------------------------ attention */

void oracle_attention(int dtype, int B, int H, int Hkv, int S_q, int S_kv, int D, int causal, const uint16_t *Q,
                      const uint16_t *K, const uint16_t *V, float *O, int q_begin, int q_end, int nthreads) {
  /* Network.swift:134-179 (S row, scale, max, exp-sum, lse, P) and 286-311 (O = P.V), per (b, h, row).
   * Query head h reads K/V head h / (H / Hkv). */
  if (q_begin < 0) q_begin = 0;
  if (q_end > S_q || q_end < 0) q_end = S_q;
  const int rows = q_end - q_begin;
  const long total = (long)B * H * rows;
  const float scale = 1.0f / sqrtf((float)D);
  const size_t ldq = (size_t)H * D; /* [B][S][H][D]: consecutive sequence positions are H*D apart */
  const size_t ldkv = (size_t)Hkv * D;
  const int group = H / Hkv;
  int nt = pick_threads(nthreads);
#pragma omp parallel num_threads(nt)
  {
    float *srow = (float *)malloc(sizeof(float) * (size_t)(S_kv > 0 ? S_kv : 1));
    float *q = (float *)malloc(sizeof(float) * (size_t)D);
    float *o = (float *)malloc(sizeof(float) * (size_t)D);
#pragma omp for schedule(dynamic, 4)
    for (long t = 0; t < total; ++t) {
      const int b = (int)(t / ((long)H * rows));
      const int h = (int)((t / rows) % H);
      const int i = q_begin + (int)(t % rows);
      const uint16_t *qp = Q + ((size_t)b * S_q + i) * ldq + (size_t)h * D;
      const uint16_t *kb = K + (size_t)b * S_kv * ldkv + (size_t)(h / group) * D;
      const uint16_t *vb = V + (size_t)b * S_kv * ldkv + (size_t)(h / group) * D;
      float *op = O + ((size_t)b * S_q + i) * ldq + (size_t)h * D;
      int ncols = S_kv;
      if (causal) {
        long lim = (long)i + (S_kv - S_q) + 1;
        ncols = lim < 0 ? 0 : (lim > S_kv ? S_kv : (int)lim);
      }
      for (int d = 0; d < D; ++d) q[d] = to_f32(dtype, qp[d]);
      for (int d = 0; d < D; ++d) o[d] = 0.0f;
      if (ncols > 0) {
        for (int j = 0; j < ncols; ++j) { /* createMatrixSRow */
          const uint16_t *kp = kb + (size_t)j * ldkv;
          float dot = 0.0f;
          for (int d = 0; d < D; ++d) dot += q[d] * to_f32(dtype, kp[d]);
          srow[j] = dot;
        }
        float maximum = -3.40282347e38f; /* -.greatestFiniteMagnitude */
        for (int j = 0; j < ncols; ++j) {
          float v = scale * srow[j];
          maximum = v > maximum ? v : maximum;
        }
        float sum = 0.0f;
        for (int j = 0; j < ncols; ++j) sum += expf(scale * srow[j] - maximum);
        const float lse = maximum + logf(sum);
        for (int j = 0; j < ncols; ++j) srow[j] = expf(scale * srow[j] - lse);
        for (int j = 0; j < ncols; ++j) { /* O[d] = sum_j P[j] * V[j][d], j ascending per d */
          const uint16_t *vp = vb + (size_t)j * ldkv;
          const float p = srow[j];
          for (int d = 0; d < D; ++d) o[d] += p * to_f32(dtype, vp[d]);
        }
      }
      for (int d = 0; d < D; ++d) op[d] = o[d];
    }
    free(srow);
    free(q);
    free(o);
  }
}

/* ------------------------------------------------------------------ convolution */

void oracle_attention_bwd(int dtype, int B, int H, int Hkv, int S_q, int S_kv, int D, int causal, const uint16_t *Q,
                          const uint16_t *K, const uint16_t *V, const uint16_t *dO, float *dQ, float *dK, float *dV,
                          float *Dterm, int bh_begin, int bh_end, int nthreads) {
  /* Per (b, h), rows i ascending (Network.swift): P row (createMatrixPRow, 151-179), O row = P.V and
   * D = O . dO (createDerivativeSRow 221-238), dP row = dO.V^T (205-218), dS = P (dP - D) * scale
   * (240-251); dQ row = dS.K, columns ascending per d (derivativeQ 376-401); dV[j] += P_j dO[i] and
   * dK[j] += dS_j Q[i], accumulated over rows in order (derivativeV 319-338, derivativeK 341-360).
   * One thread owns one (b, K/V head): its query heads h = hk * group + 0 .. group - 1 in order, each
   * with rows ascending, so every sum keeps the reference's order (with Hkv == H, one (b, h)).
   * [bh_begin, bh_end) ranges over the B * Hkv (batch, K/V head) pairs. */
  if (bh_begin < 0) bh_begin = 0;
  if (bh_end < 0 || bh_end > B * Hkv) bh_end = B * Hkv;
  const float scale = 1.0f / sqrtf((float)D);
  const size_t ldq = (size_t)H * D, ldkv = (size_t)Hkv * D;
  const int group = H / Hkv;
  int nt = pick_threads(nthreads);
  if (nt > bh_end - bh_begin) nt = bh_end - bh_begin > 0 ? bh_end - bh_begin : 1;
#pragma omp parallel num_threads(nt)
  {
    float *srow = (float *)malloc(sizeof(float) * (size_t)(S_kv > 0 ? S_kv : 1));
    float *dprow = (float *)malloc(sizeof(float) * (size_t)(S_kv > 0 ? S_kv : 1));
    float *q = (float *)malloc(sizeof(float) * (size_t)D);
    float *go = (float *)malloc(sizeof(float) * (size_t)D);
    float *o = (float *)malloc(sizeof(float) * (size_t)D);
    float *dq = (float *)malloc(sizeof(float) * (size_t)D);
    float *kf = (float *)malloc(sizeof(float) * (size_t)S_kv * D + 1);
    float *vf = (float *)malloc(sizeof(float) * (size_t)S_kv * D + 1);
    float *dk = (float *)malloc(sizeof(float) * (size_t)S_kv * D + 1);
    float *dv = (float *)malloc(sizeof(float) * (size_t)S_kv * D + 1);
#pragma omp for schedule(dynamic, 1)
    for (int bh = bh_begin; bh < bh_end; ++bh) {
      const int b = bh / Hkv, hk = bh % Hkv;
      const uint16_t *kb = K + (size_t)b * S_kv * ldkv + (size_t)hk * D;
      const uint16_t *vb = V + (size_t)b * S_kv * ldkv + (size_t)hk * D;
      for (int j = 0; j < S_kv; ++j)
        for (int d = 0; d < D; ++d) {
          kf[(size_t)j * D + d] = to_f32(dtype, kb[(size_t)j * ldkv + d]);
          vf[(size_t)j * D + d] = to_f32(dtype, vb[(size_t)j * ldkv + d]);
        }
      memset(dk, 0, sizeof(float) * (size_t)S_kv * D);
      memset(dv, 0, sizeof(float) * (size_t)S_kv * D);
      for (int h = hk * group; h < hk * group + group; ++h)
      for (int i = 0; i < S_q; ++i) {
        const uint16_t *qp = Q + ((size_t)b * S_q + i) * ldq + (size_t)h * D;
        const uint16_t *gp = dO + ((size_t)b * S_q + i) * ldq + (size_t)h * D;
        int ncols = S_kv;
        if (causal) {
          long lim = (long)i + (S_kv - S_q) + 1;
          ncols = lim < 0 ? 0 : (lim > S_kv ? S_kv : (int)lim);
        }
        for (int d = 0; d < D; ++d) {
          q[d] = to_f32(dtype, qp[d]);
          go[d] = to_f32(dtype, gp[d]);
          o[d] = 0.0f;
          dq[d] = 0.0f;
        }
        float term_d = 0.0f;
        if (ncols > 0) {
          for (int j = 0; j < ncols; ++j) { /* S row */
            const float *kp = kf + (size_t)j * D;
            float dot = 0.0f;
            for (int d = 0; d < D; ++d) dot += q[d] * kp[d];
            srow[j] = dot;
          }
          float maximum = -3.40282347e38f;
          for (int j = 0; j < ncols; ++j) {
            float v = scale * srow[j];
            maximum = v > maximum ? v : maximum;
          }
          float sum = 0.0f;
          for (int j = 0; j < ncols; ++j) sum += expf(scale * srow[j] - maximum);
          const float lse = maximum + logf(sum);
          for (int j = 0; j < ncols; ++j) srow[j] = expf(scale * srow[j] - lse); /* P row */
          for (int j = 0; j < ncols; ++j) { /* O = P.V, j ascending per d */
            const float *vp = vf + (size_t)j * D;
            const float p = srow[j];
            for (int d = 0; d < D; ++d) o[d] += p * vp[d];
          }
          for (int d = 0; d < D; ++d) term_d += o[d] * go[d];
          for (int j = 0; j < ncols; ++j) { /* dP row = dO . V^T */
            const float *vp = vf + (size_t)j * D;
            float dot = 0.0f;
            for (int d = 0; d < D; ++d) dot += go[d] * vp[d];
            dprow[j] = dot;
          }
          for (int j = 0; j < ncols; ++j) { /* dS row; dQ, dK, dV updates */
            float ds = srow[j] * (dprow[j] - term_d);
            ds *= scale;
            const float p = srow[j];
            const float *kp = kf + (size_t)j * D;
            float *dkp = dk + (size_t)j * D, *dvp = dv + (size_t)j * D;
            for (int d = 0; d < D; ++d) {
              dq[d] += ds * kp[d];
              dvp[d] += p * go[d];
              dkp[d] += ds * q[d];
            }
          }
        }
        if (Dterm) Dterm[((size_t)b * H + h) * S_q + i] = term_d;
        float *dqp = dQ + ((size_t)b * S_q + i) * ldq + (size_t)h * D;
        for (int d = 0; d < D; ++d) dqp[d] = dq[d];
      }
      for (int j = 0; j < S_kv; ++j) {
        float *dkp = dK + ((size_t)b * S_kv + j) * ldkv + (size_t)hk * D;
        float *dvp = dV + ((size_t)b * S_kv + j) * ldkv + (size_t)hk * D;
        for (int d = 0; d < D; ++d) {
          dkp[d] = dk[(size_t)j * D + d];
          dvp[d] = dv[(size_t)j * D + d];
        }
      }
    }
    free(srow);
    free(dprow);
    free(q);
    free(go);
    free(o);
    free(dq);
    free(kf);
    free(vf);
    free(dk);
    free(dv);
  }
}

int oracle_conv_out_d(const oracle_conv_dims *d) {
  return (d->D + d->PF + d->PBk - ((d->KD - 1) * d->DZ + 1)) / d->SZ + 1;
}
int oracle_conv_out_h(const oracle_conv_dims *d) {
  return (d->H + d->PT + d->PB - ((d->KH - 1) * d->DY + 1)) / d->SY + 1;
}
int oracle_conv_out_w(const oracle_conv_dims *d) {
  return (d->W + d->PL + d->PR - ((d->KW - 1) * d->DX + 1)) / d->SX + 1;
}

void oracle_conv(const oracle_conv_dims *d, const uint16_t *x, const uint16_t *w, const uint16_t *bias, float *y,
                 long row_begin, long row_end, int nthreads) {
  /* ConvolutionShared.swift:4994-5068: for each output (n, oz, oh, ow, oc): sum over kd, kh, kw, ic of
   * a * w, skipping out-of-bounds taps; bias added after the full sum (5083-5093). Depth padding
   * (PF) is this build's extension; PF = 0 restates the reference exactly. */
  const int OD = oracle_conv_out_d(d), OH = oracle_conv_out_h(d), OW = oracle_conv_out_w(d);
  const int C = d->C, O = d->O;
  const long rows = (long)d->N * OD * OH;
  if (row_begin < 0) row_begin = 0;
  if (row_end < 0 || row_end > rows) row_end = rows;
  const size_t wcount = (size_t)d->KD * d->KH * d->KW * C * O;
  float *wf = (float *)malloc(sizeof(float) * (wcount ? wcount : 1));
  for (size_t i = 0; i < wcount; ++i) wf[i] = to_f32(ORACLE_F16, w[i]);
  int nt = pick_threads(nthreads);
#pragma omp parallel num_threads(nt)
  {
    float *acc = (float *)malloc(sizeof(float) * (size_t)O);
#pragma omp for schedule(static)
    for (long r = row_begin; r < row_end; ++r) {
      const int n = (int)(r / ((long)OD * OH));
      const int oz = (int)((r / OH) % OD);
      const int oh = (int)(r % OH);
      for (int ow = 0; ow < OW; ++ow) {
        for (int oc = 0; oc < O; ++oc) acc[oc] = 0.0f;
        for (int kd = 0; kd < d->KD; ++kd) {
          const int iz = oz * d->SZ + kd * d->DZ - d->PF;
          if (iz < 0 || iz >= d->D) continue;
          for (int kh = 0; kh < d->KH; ++kh) {
            const int ih = oh * d->SY + kh * d->DY - d->PT;
            if (ih < 0 || ih >= d->H) continue;
            for (int kw = 0; kw < d->KW; ++kw) {
              const int iw = ow * d->SX + kw * d->DX - d->PL;
              if (iw < 0 || iw >= d->W) continue;
              const uint16_t *xp = x + ((((size_t)n * d->D + iz) * d->H + ih) * d->W + iw) * C;
              const float *wp = wf + (((size_t)kd * d->KH + kh) * d->KW + kw) * C * O;
              for (int ic = 0; ic < C; ++ic) {
                const float a = oracle_f16_to_f32(xp[ic]);
                const float *wr = wp + (size_t)ic * O;
                for (int oc = 0; oc < O; ++oc) acc[oc] += a * wr[oc];
              }
            }
          }
        }
        float *yp = y + ((((size_t)n * OD + oz) * OH + oh) * OW + ow) * O;
        for (int oc = 0; oc < O; ++oc) yp[oc] = bias ? acc[oc] + oracle_f16_to_f32(bias[oc]) : acc[oc];
      }
    }
    free(acc);
  }
  free(wf);
}

void oracle_permute_oidhw_to_dhwio(const uint16_t *src, uint16_t *dst, int O, int C, int KD, int KH, int KW) {
  /* ConvolutionShared.swift:4606-4627: destination index gid decomposed as (kd, kh, kw, ic, oc) with
   * oc fastest; source index ((((oc * C + ic) * KD + kd) * KH + kh) * KW) + kw. */
  const size_t count = (size_t)O * C * KD * KH * KW;
  for (size_t gid = 0; gid < count; ++gid) {
    size_t linear = gid;
    const size_t oc = linear % (size_t)O;
    linear /= (size_t)O;
    const size_t ic = linear % (size_t)C;
    linear /= (size_t)C;
    const size_t kw = linear % (size_t)KW;
    linear /= (size_t)KW;
    const size_t kh = linear % (size_t)KH;
    linear /= (size_t)KH;
    const size_t kd = linear;
    dst[gid] = src[((((oc * C + ic) * KD + kd) * KH + kh) * KW) + kw];
  }
}
