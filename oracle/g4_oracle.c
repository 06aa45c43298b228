/* g4_oracle.c -- CPU restatement of the reference's speculative-verify path.
 *
 * TEST INFRASTRUCTURE: the checker for the HIP product and the "port" CPU
 * baseline.  Never linked by the product.  Compiled with -ffp-contract=off;
 * every fused multiply-add below is explicit and mirrors an FMA in the
 * reference (an intrinsic, or a contraction GCC makes at -O3
 * -march=x86-64-v3 under its default -ffp-contract=fast).
 *
 * Citations are to dayaswaroopchavali/gemma4-e2b-laptop-cpu:
 *   W = engine/w4g32_avx2.h, A8 = engine/w4a8_avx2.h,
 *   X3 = engine/bf16_exp3_head.h, E = engine/gemma4_engine.cpp.
 */
#include "g4_oracle.h"
#include "g4_rng.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* scalar numerics                                                          */
/* ------------------------------------------------------------------------ */

/* E:34 f2bf: round-to-nearest-even to bf16; NaN keeps a quiet payload */
uint16_t g4o_f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* W:15 bf16_to_f32 */
float g4o_bf2f(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* E:35 r16 and E:37-42 rbf8 (identical on every non-NaN input) */
float g4o_r16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xFFFF0000u;
  float r;
  memcpy(&r, &u, 4);
  return r;
}

static inline float fminmax_clamp(float x) {
  /* _mm256_max_ps(x, -87.3f) then _mm256_min_ps(., 88.3f): the second operand is
   * returned when the comparison is false (NaN propagates as the constant) */
  float a = (x > -87.3f) ? x : -87.3f;
  return (a < 88.3f) ? a : 88.3f;
}

/* E:43-53 exp8, one lane: Cephes expf (S. L. Moshier) with the engine's FMA order */
float g4o_exp8(float x) {
  x = fminmax_clamp(x);
  float fx = floorf(fmaf(x, 1.44269504088896341f, 0.5f));
  x = fmaf(-fx, 0.693359375f, x);
  x = fmaf(-fx, -2.12194440e-4f, x);
  float z = x * x;
  float y = 1.9875691500E-4f;
  y = fmaf(y, x, 1.3981999507E-3f);
  y = fmaf(y, x, 8.3334519073E-3f);
  y = fmaf(y, x, 4.1665795894E-2f);
  y = fmaf(y, x, 1.6666665459E-1f);
  y = fmaf(y, x, 5.0000001201E-1f);
  y = fmaf(y, z, x + 1.0f);
  int32_t n = ((int32_t)fx + 127) << 23; /* cvttps: truncation of an integral value */
  float p;
  memcpy(&p, &n, 4);
  return y * p;
}

/* E:54-60 gelu8, one lane: 0.5 x (1 + tanh(u)), tanh(u) = 1 - 2 / (exp(2u) + 1) */
float g4o_gelu8(float x) {
  float x3 = (x * x) * x;
  float u = 0.7978845608028654f * fmaf(0.044715f, x3, x);
  float e = g4o_exp8(2.0f * u);
  float th = 1.0f - 2.0f / (e + 1.0f);
  return (0.5f * x) * (1.0f + th);
}

void g4o_vec_exp8(const float* x, int n, float* y) { for (int i = 0; i < n; ++i) y[i] = g4o_exp8(x[i]); }
void g4o_vec_gelu8(const float* x, int n, float* y) { for (int i = 0; i < n; ++i) y[i] = g4o_gelu8(x[i]); }

/* E:326-343 ss_avx2: four 4-lane double accumulators over steps of 16, then
 * ((s0+s1)+(s2+s3)) lane-wise and (l0+l2)+(l1+l3). n % 16 == 0. */
double g4o_sumsq(const float* x, int n) {
  double s[4][4] = {{0}};
  for (int i = 0; i < n; i += 16)
    for (int k = 0; k < 4; ++k)
      for (int l = 0; l < 4; ++l) {
        double d = (double)x[i + 4 * k + l];
        s[k][l] = fma(d, d, s[k][l]);
      }
  double a[4];
  for (int l = 0; l < 4; ++l) a[l] = (s[0][l] + s[1][l]) + (s[2][l] + s[3][l]);
  return (a[0] + a[2]) + (a[1] + a[3]);
}

/* E:345 r = 1 / sqrtf((float)(ss / n) + eps), eps = 1e-6 */
float g4o_rms_inv(const float* x, int n) {
  double ss = g4o_sumsq(x, n);
  return 1.0f / sqrtf((float)(ss / n) + 1e-6f);
}

/* E:344-352 rms: y = (x * r) * w  (w == NULL: y = x * r) */
void g4o_rms(const float* x, const float* w, int n, float* y) {
  float r = g4o_rms_inv(x, n);
  for (int i = 0; i < n; ++i) y[i] = w ? (x[i] * r) * w[i] : x[i] * r;
}

/* E:353-361 rms_r16_inplace */
void g4o_rms_r16_inplace(float* x, const float* w, int n) {
  float r = g4o_rms_inv(x, n);
  for (int i = 0; i < n; ++i) x[i] = g4o_r16(w ? (x[i] * r) * w[i] : x[i] * r);
}

/* E:394-402 rope_avx2 (NeoX halves): h[j] = u c - (w s), h[j+hh] = w c + (u s), both fused */
void g4o_rope(float* h, const float* cs, const float* sn, int hd) {
  const int hh = hd / 2;
  for (int j = 0; j < hh; ++j) {
    float u = h[j], w = h[j + hh], c = cs[j], s = sn[j];
    float ws = w * s, us = u * s;
    h[j] = fmaf(u, c, -ws);
    h[j + hh] = fmaf(w, c, us);
  }
}

/* E:1246-1247 RoPE tables: inv_j = 1/theta^(2j/hd) for j < rot, 0 beyond; cos/sin in double */
void g4o_rope_tables(int ctx, int hd, double theta, double rot_frac, float* cs, float* sn) {
  int ra = (int)(hd * rot_frac) / 2;
  for (int p = 0; p < ctx; ++p)
    for (int j = 0; j < hd / 2; ++j) {
      double inv = j < ra ? 1.0 / pow(theta, (2.0 * j) / hd) : 0.0;
      double ang = p * inv;
      cs[(size_t)p * hd / 2 + j] = (float)cos(ang);
      sn[(size_t)p * hd / 2 + j] = (float)sin(ang);
    }
}

/* E:455, E:1409 cap(s) = r16(30 tanh(s / 30)) */
float g4o_cap(float s) { return g4o_r16(30.0f * tanhf(s / 30.0f)); }

/* E:454-459 calc_thr_fast == E:1410-1414 calc_thr: 40-step bisection for the smallest z
 * with cap(r16 z) == cap(r16 L), minus 0.25 */
float g4o_calc_thr(float L) {
  float Lr = g4o_r16(L), cmL = g4o_cap(Lr), lo = Lr - 64.0f, hi = Lr;
  for (int it = 0; it < 40; ++it) {
    float mid = 0.5f * (lo + hi);
    if (g4o_cap(g4o_r16(mid)) == cmL) hi = mid;
    else lo = mid;
  }
  return hi - 0.25f;
}

/* W:41-44 hsum / X3:78-81 hsum8: ((r0+r4)+(r1+r5))+((r2+r6)+(r3+r7)) */
static inline float hsum8(const float* r) {
  float a0 = r[0] + r[4], a1 = r[1] + r[5], a2 = r[2] + r[6], a3 = r[3] + r[7];
  return (a0 + a1) + (a2 + a3);
}

/* ------------------------------------------------------------------------ */
/* W4G32                                                                     */
/* ------------------------------------------------------------------------ */

/* W:20-23 prep_x (== E:180-224 XP::prep / prep_x_avx2 / prep_g32_from_vecs):
 * even/odd split and sequential per-32 group sums */
void g4o_prep_x(const float* x, int K, float* xe, float* xo, float* gs) {
  for (int i = 0; i < K / 2; ++i) {
    xe[i] = x[2 * i];
    xo[i] = x[2 * i + 1];
  }
  for (int g = 0; g < K / 32; ++g) {
    float s = 0;
    for (int i = 0; i < 32; ++i) s += x[g * 32 + i];
    gs[g] = s;
  }
}

/* W:64-96 gemm_rows_tile<MT> for M rows (xe/xo rows of K/2, gs rows of K/32).
 * Per (m, n), lane j of 8: a = l0*xe[j]; a = fma(l1, xe[8+j], a); a = fma(h0, xo[j], a);
 * a = fma(h1, xo[8+j], a); row_j = fma(a, sc, row_j); off = fma(sc, gs[g], off) (GCC
 * contraction of `off += sc * gsum`); y = hsum(row) - 8 off. */
void g4o_w4g32_rows(const uint8_t* W, const uint16_t* S, const float* xe, const float* xo,
                    const float* gs, int K, int M, int n0, int n1, float* Y, int ldy) {
  const int G = K / 32;
  const size_t rb = (size_t)K / 2;
  for (int mb = 0; mb < M; mb += 64) {
    const int MT = (M - mb) < 64 ? (M - mb) : 64;
#pragma omp parallel for schedule(static)
    for (int n = n0; n < n1; ++n) {
      float row[64][8], off[64];
      const uint8_t* w = W + (size_t)n * rb;
      const uint16_t* s = S + (size_t)n * G;
      for (int m = 0; m < MT; ++m) {
        off[m] = 0.f;
        for (int j = 0; j < 8; ++j) row[m][j] = 0.f;
      }
      for (int g = 0; g < G; ++g) {
        const uint8_t* v = w + (size_t)g * 16;
        const float sc = g4o_bf2f(s[g]);
        float l0[8], l1[8], h0[8], h1[8];
        for (int j = 0; j < 8; ++j) {
          l0[j] = (float)(v[j] & 15);
          l1[j] = (float)(v[8 + j] & 15);
          h0[j] = (float)(v[j] >> 4);
          h1[j] = (float)(v[8 + j] >> 4);
        }
        for (int m = 0; m < MT; ++m) {
          const float* pe = xe + (size_t)(mb + m) * (K / 2) + g * 16;
          const float* po = xo + (size_t)(mb + m) * (K / 2) + g * 16;
          for (int j = 0; j < 8; ++j) {
            float a = l0[j] * pe[j];
            a = fmaf(l1[j], pe[8 + j], a);
            a = fmaf(h0[j], po[j], a);
            a = fmaf(h1[j], po[8 + j], a);
            row[m][j] = fmaf(a, sc, row[m][j]);
          }
          off[m] = fmaf(sc, gs[(size_t)(mb + m) * G + g], off[m]);
        }
      }
      for (int m = 0; m < MT; ++m) Y[(size_t)(mb + m) * ldy + n] = hsum8(row[m]) - 8.f * off[m];
    }
  }
}

/* E:241-255 lin_task / E:310-317 lin1: prep each row, all N outputs (the result is
 * independent of the 4-row tiling and of the thread split) */
void g4o_w4g32_gemm(const uint8_t* W, const uint16_t* S, const float* X, int M, int N, int K,
                    float* Y) {
  float* xe = (float*)malloc(sizeof(float) * (size_t)M * K / 2);
  float* xo = (float*)malloc(sizeof(float) * (size_t)M * K / 2);
  float* gs = (float*)malloc(sizeof(float) * (size_t)M * K / 32);
  for (int m = 0; m < M; ++m)
    g4o_prep_x(X + (size_t)m * K, K, xe + (size_t)m * K / 2, xo + (size_t)m * K / 2,
               gs + (size_t)m * K / 32);
  g4o_w4g32_rows(W, S, xe, xo, gs, K, M, 0, N, Y, N);
  free(xe);
  free(xo);
  free(gs);
}

/* ------------------------------------------------------------------------ */
/* prompt lookup                                                             */
/* ------------------------------------------------------------------------ */

/* E:1624-1628: scan i = L-n-1 down to 0 for seq[i .. i+n) == seq[L-n .. L); at the first hit
 * copy seq[i+n+j] for j < maxlen while i+n+j < L */
int g4o_prompt_lookup(const int32_t* seq, int L, int n, int maxlen, int32_t* drafts) {
  int nd = 0;
  if (n <= 0 || L <= n) return 0;
  for (int i = L - n - 1; i >= 0; --i) {
    int eq = 1;
    for (int t = 0; t < n; ++t)
      if (seq[i + t] != seq[L - n + t]) {
        eq = 0;
        break;
      }
    if (eq) {
      for (int j = 0; j < maxlen && i + n + j < L; ++j) drafts[nd++] = seq[i + n + j];
      break;
    }
  }
  return nd;
}

/* ------------------------------------------------------------------------ */
/* W4A8                                                                      */
/* ------------------------------------------------------------------------ */

/* A8:30-42 quant: per (row, 32-group) sx = amax/127, inv = 1/sx, q = RNE(x*inv) saturated
 * to int8, sum = sum of the unsaturated integers */
void g4o_w4a8_quant(const float* X, int M, int K, int8_t* q, float* sx, int32_t* sum) {
  const int G = K / 32;
  for (int m = 0; m < M; ++m)
    for (int g = 0; g < G; ++g) {
      const float* p = X + (size_t)m * K + g * 32;
      float amax = 0.f;
      for (int i = 0; i < 32; ++i) {
        float a = fabsf(p[i]);
        amax = (amax > a) ? amax : a;
      }
      float s = amax / 127.0f, inv = s > 0 ? 1.0f / s : 0.0f;
      int32_t tot = 0;
      for (int i = 0; i < 32; ++i) {
        float v = nearbyintf(p[i] * inv);
        int32_t iv = (int32_t)v;
        tot += iv;
        if (iv > 127) iv = 127;
        if (iv < -128) iv = -128;
        q[(size_t)m * K + g * 32 + i] = (int8_t)iv;
      }
      sx[(size_t)m * G + g] = s;
      sum[(size_t)m * G + g] = tot;
    }
}

/* A8:46-61 tile<MT> (weights in the original [N][K/2] layout; the 8-row repack of A8:18-27
 * only reorders the exact integer dot): per (m, n, g) a32 = sum u*xq - 8 sum(xq) (exact,
 * no int16 overflow: |partial| <= 30,480), row = fma((float)a32, sw*sx, row) */
void g4o_w4a8_gemm(const uint8_t* W, const uint16_t* S, const float* X, int M, int N, int K,
                   float* Y) {
  const int G = K / 32;
  int8_t* q = (int8_t*)malloc((size_t)M * K);
  float* sx = (float*)malloc(sizeof(float) * (size_t)M * G);
  int32_t* sm = (int32_t*)malloc(sizeof(int32_t) * (size_t)M * G);
  g4o_w4a8_quant(X, M, K, q, sx, sm);
  /* every output is its own sequential chain: outputs split over threads freely */
#pragma omp parallel for collapse(2) schedule(static)
  for (int m = 0; m < M; ++m)
    for (int n = 0; n < N; ++n) {
      float row = 0.f;
      for (int g = 0; g < G; ++g) {
        int32_t a = 0;
        for (int i = 0; i < 32; ++i) {
          int k = g * 32 + i;
          uint8_t b = W[(size_t)n * (K / 2) + k / 2];
          int u = (k & 1) ? (b >> 4) : (b & 15);
          a += u * (int32_t)q[(size_t)m * K + k];
        }
        a -= 8 * sm[(size_t)m * G + g];
        float sc = g4o_bf2f(S[(size_t)n * G + g]) * sx[(size_t)m * G + g];
        row = fmaf((float)a, sc, row);
      }
      Y[(size_t)m * N + n] = row;
    }
  free(q);
  free(sx);
  free(sm);
}

/* ------------------------------------------------------------------------ */
/* exp3-packed bf16 head                                                     */
/* ------------------------------------------------------------------------ */

/* E:1232-1234 codebook: the 8 most frequent exponents, stable order on ties */
void g4o_exp3_codebook(const uint16_t* E, int64_t n, uint8_t cb8[8]) {
  int64_t hist[256];
  memset(hist, 0, sizeof hist);
  for (int64_t i = 0; i < n; ++i) hist[(E[i] >> 7) & 0xFF]++;
  int ord[256];
  for (int i = 0; i < 256; ++i) ord[i] = i;
  /* stable insertion sort by count, descending */
  for (int i = 1; i < 256; ++i) {
    int v = ord[i], j = i;
    while (j > 0 && hist[ord[j - 1]] < hist[v]) {
      ord[j] = ord[j - 1];
      --j;
    }
    ord[j] = v;
  }
  for (int i = 0; i < 8; ++i) cb8[i] = (uint8_t)ord[i];
}

/* X3:34-39 codebook index: exact match, else the first nearest exponent */
static inline int exp3_index(const uint8_t cb8[8], int e, int* exc) {
  for (int i = 0; i < 8; ++i)
    if (cb8[i] == e) {
      *exc = 0;
      return i;
    }
  int best = 0, bd = 1 << 30;
  for (int i = 0; i < 8; ++i) {
    int dd = abs((int)cb8[i] - e);
    if (dd < bd) {
      bd = dd;
      best = i;
    }
  }
  *exc = 1;
  return best;
}

int64_t g4o_exp3_count(const uint16_t* W, int N, int K, const uint8_t cb8[8], int64_t* exc_ptr) {
  exc_ptr[0] = 0;
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; ++n) {
    int64_t c = 0;
    for (int k = 0; k < K; ++k) {
      int e = (W[(size_t)n * K + k] >> 7) & 0xFF, exc;
      exp3_index(cb8, e, &exc);
      c += exc;
    }
    exc_ptr[n + 1] = c;
  }
  for (int n = 0; n < N; ++n) exc_ptr[n + 1] += exc_ptr[n];
  return exc_ptr[N];
}

/* X3:26-49 pack: 32 B sign|mant7, then three 4-B exponent-index bit planes per 32-group;
 * exceptions store the nearest codebook exponent plus an exact fp32 delta (CSR by row) */
void g4o_exp3_pack(const uint16_t* W, int N, int K, const uint8_t cb8[8], uint8_t* data,
                   const int64_t* exc_ptr, uint16_t* exc_col, float* exc_delta) {
  const int G = K / 32;
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; ++n) {
    int64_t e_at = exc_ptr[n];
    for (int g = 0; g < G; ++g) {
      uint8_t* d = data + ((size_t)n * G + g) * 44;
      uint32_t pl[3] = {0, 0, 0};
      for (int j = 0; j < 32; ++j) {
        uint16_t w = W[(size_t)n * K + g * 32 + j];
        int sign = w >> 15, e = (w >> 7) & 0xFF, mnt = w & 0x7F, exc;
        int idx = exp3_index(cb8, e, &exc);
        if (exc) {
          uint16_t dec = (uint16_t)((sign << 15) | (cb8[idx] << 7) | mnt);
          exc_col[e_at] = (uint16_t)(g * 32 + j);
          exc_delta[e_at] = g4o_bf2f(w) - g4o_bf2f(dec);
          ++e_at;
        }
        d[j] = (uint8_t)((sign << 7) | mnt);
        for (int k = 0; k < 3; ++k) pl[k] |= (uint32_t)((idx >> k) & 1) << j;
      }
      memcpy(d + 32, pl, 12);
    }
  }
}

/* X3:59-76 decode_group: the 32 bf16 weights of one 44-byte group, in element order */
static inline void exp3_group(const uint8_t* d, const uint8_t cb8[8], float* w) {
  uint32_t p0, p1, p2;
  memcpy(&p0, d + 32, 4);
  memcpy(&p1, d + 36, 4);
  memcpy(&p2, d + 40, 4);
  for (int j = 0; j < 32; ++j) {
    int idx = ((p0 >> j) & 1) | (((p1 >> j) & 1) << 1) | (((p2 >> j) & 1) << 2);
    uint8_t sm = d[j];
    uint16_t b = (uint16_t)(((sm & 0x80) << 8) | ((uint16_t)cb8[idx] << 7) | (sm & 0x7F));
    w[j] = g4o_bf2f(b);
  }
}

/* X3:83-107 rows_tile (== E:540-571 resc_task body): lane j accumulates weights
 * j, 16+j, 8+j, 24+j of every group by FMA; y = hsum8; then y = fma(delta, x[col], y)
 * over the row's exceptions in order (GCC contraction of `y += delta * x`). */
float g4o_exp3_dot(const uint8_t* data, const uint8_t cb8[8], const int64_t* exc_ptr,
                   const uint16_t* exc_col, const float* exc_delta, int K, int n, const float* x) {
  const int G = K / 32;
  const uint8_t* row = data + (size_t)n * G * 44;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0}, w[32];
  for (int g = 0; g < G; ++g) {
    exp3_group(row + (size_t)g * 44, cb8, w);
    const float* xg = x + g * 32;
    for (int j = 0; j < 8; ++j) {
      acc[j] = fmaf(w[j], xg[j], acc[j]);
      acc[j] = fmaf(w[16 + j], xg[16 + j], acc[j]);
      acc[j] = fmaf(w[8 + j], xg[8 + j], acc[j]);
      acc[j] = fmaf(w[24 + j], xg[24 + j], acc[j]);
    }
  }
  float y = hsum8(acc);
  for (int64_t e = exc_ptr[n]; e < exc_ptr[n + 1]; ++e) y = fmaf(exc_delta[e], x[exc_col[e]], y);
  return y;
}

/* X3:109-117 gemm / E:573-579 head_task: Y[m][n] for all rows */
void g4o_exp3_gemm(const uint8_t* data, const uint8_t cb8[8], const int64_t* exc_ptr,
                   const uint16_t* exc_col, const float* exc_delta, int N, int K, const float* X,
                   int M, float* Y) {
  for (int m = 0; m < M; ++m)
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n)
      Y[(size_t)m * N + n] =
          g4o_exp3_dot(data, cb8, exc_ptr, exc_col, exc_delta, K, n, X + (size_t)m * K);
}

/* ------------------------------------------------------------------------ */
/* certified head screen                                                    */
/* ------------------------------------------------------------------------ */

/* E:1236-1243 screen build: per 32-group sb = f2bf(amax/7); u = clamp(nearbyintf(w/sc),-8,7)+8
 * (even element in the low nibble); e2 += d*d, w2 += w*w in double; coef = (float)fma(1e-4,
 * sqrt(w2), sqrt(e2)) -- GCC contracts `sqrt(e2) + 1e-4 * sqrt(w2)` into one FMA. */
void g4o_screen_build(const uint16_t* E, int N, int K, uint8_t* Wq, uint16_t* Sq, float* coef) {
  const int G = K / 32;
#pragma omp parallel for schedule(static)
  for (int n = 0; n < N; ++n) {
    double e2 = 0, w2 = 0;
    for (int g = 0; g < G; ++g) {
      float amax = 0, w[32];
      for (int i = 0; i < 32; ++i) {
        w[i] = g4o_bf2f(E[(size_t)n * K + g * 32 + i]);
        float a = fabsf(w[i]);
        amax = (amax < a) ? a : amax; /* std::max(amax, |w|) */
      }
      uint16_t sb = g4o_f2bf(amax / 7.0f);
      float sc = g4o_bf2f(sb);
      Sq[(size_t)n * G + g] = sb;
      int qv[32];
      for (int i = 0; i < 32; ++i) {
        int v = sc > 0 ? (int)nearbyintf(w[i] / sc) : 0;
        v = v < -8 ? -8 : (v > 7 ? 7 : v);
        qv[i] = v + 8;
        double d = fma(-(double)v, (double)sc, (double)w[i]);
        e2 = fma(d, d, e2);
        w2 = fma((double)w[i], (double)w[i], w2);
      }
      for (int i = 0; i < 16; ++i)
        Wq[(size_t)n * (K / 2) + g * 16 + i] = (uint8_t)(qv[2 * i] | (qv[2 * i + 1] << 4));
    }
    coef[n] = (float)fma(1e-4, sqrt(w2), sqrt(e2));
  }
}

/* Single-thread replay of E:460-538 screen_task's prefilter list, only to report whether the
 * reference (one worker) overflows its 16,384-entry list.  Chunks of 64 rows; the running
 * 8-lane max of L is compared against cur_best + 0.05 after each chunk. */
static int screen_ref_overflow(const float* U, const float* L, int V, float seedL) {
  float cur = seedL, thr = g4o_calc_thr(cur) - 1e-4f;
  float vmx[8];
  for (int l = 0; l < 8; ++l) vmx[l] = -1e30f;
  int cnt = 0;
  for (int n0 = 0; n0 < V; n0 += 64) {
    for (int i = n0; i < n0 + 64 && i < V; ++i) {
      int l = (i - n0) & 7;
      vmx[l] = (vmx[l] > L[i]) ? vmx[l] : L[i];
      if (U[i] >= thr) {
        if (cnt < 16384) ++cnt;
        else return 1;
      }
    }
    float mx = vmx[0];
    int any = 0;
    for (int l = 0; l < 8; ++l) any |= vmx[l] > cur + 0.05f;
    if (any) {
      for (int l = 1; l < 8; ++l) mx = (mx < vmx[l]) ? vmx[l] : mx;
      if (mx > cur + 0.05f) {
        cur = mx;
        thr = g4o_calc_thr(mx) - 1e-4f;
      }
    }
  }
  return 0;
}

/* One head row (E:1415-1498 with Mh = 1): screen s = W4G32(screen, h); L = s - c|h|,
 * U = c|h| + s (both fused); thr = calc_thr(max L); survivors {U >= thr} ascending;
 * rescore r16(exp3 dot); G = first survivor with v >= mx - 2 and cap(v) == cap(mx).
 * More than `limit` survivors (or the single-thread list overflow) -> full head, r16,
 * lowest index with the same tie rule. */
void g4o_head_row(const float* h, int V, int K, const uint8_t* Wq, const uint16_t* Sq,
                  const float* coef, const uint8_t* data, const uint8_t cb8[8],
                  const int64_t* exc_ptr, const uint16_t* exc_col, const float* exc_delta,
                  const int* seeds, int nseeds, int limit, int* surv, float* sval, int cap_surv,
                  g4o_head_info* info) {
  float* xe = (float*)malloc(sizeof(float) * K / 2);
  float* xo = (float*)malloc(sizeof(float) * K / 2);
  float* gs = (float*)malloc(sizeof(float) * K / 32);
  float* s = (float*)malloc(sizeof(float) * (size_t)V);
  float* U = (float*)malloc(sizeof(float) * (size_t)V);
  float* L = (float*)malloc(sizeof(float) * (size_t)V);
  g4o_prep_x(h, K, xe, xo, gs);
  float hn = (float)sqrt(g4o_sumsq(h, K));
  g4o_w4g32_rows(Wq, Sq, xe, xo, gs, K, 1, 0, V, s, V);
  float Lmax = -1e30f;
  for (int n = 0; n < V; ++n) {
    L[n] = fmaf(-coef[n], hn, s[n]);
    U[n] = fmaf(coef[n], hn, s[n]);
    Lmax = (Lmax < L[n]) ? L[n] : Lmax;
  }
  float seedL = -1e30f;
  for (int i = 0; i < nseeds; ++i) {
    int n = seeds[i];
    if (n < 0 || n >= V) continue;
    seedL = (seedL < L[n]) ? L[n] : seedL;
  }
  info->ref_overflow = screen_ref_overflow(U, L, V, seedL);
  float thr = g4o_calc_thr(Lmax);
  int ns = 0;
  for (int n = 0; n < V; ++n)
    if (U[n] >= thr) {
      if (ns < cap_surv) surv[ns] = n;
      ++ns;
    }
  info->Lmax = Lmax;
  info->thr = thr;
  info->nsurv = ns;
  info->fallback = (ns > limit || info->ref_overflow) ? 1 : 0;
  int best = -1;
  float mx = -1e30f;
  /* the survivors' exact logits are reported whenever the list fits, even on fallback */
  for (int i = 0; i < ns && i < cap_surv && ns <= limit; ++i) {
    float v = g4o_r16(g4o_exp3_dot(data, cb8, exc_ptr, exc_col, exc_delta, K, surv[i], h));
    sval[i] = v;
    mx = (mx < v) ? v : mx;
  }
  if (!info->fallback) {
    float cm = g4o_cap(mx);
    for (int i = 0; i < ns && i < cap_surv; ++i)
      if (sval[i] >= mx - 2.0f && g4o_cap(sval[i]) == cm) {
        best = surv[i];
        break;
      }
  } else {
    float* lg = s; /* reuse */
#pragma omp parallel for schedule(static)
    for (int n = 0; n < V; ++n) lg[n] = g4o_r16(g4o_exp3_dot(data, cb8, exc_ptr, exc_col, exc_delta, K, n, h));
    for (int n = 0; n < V; ++n) mx = (mx < lg[n]) ? lg[n] : mx;
    float cm = g4o_cap(mx);
    for (int n = 0; n < V; ++n)
      if (lg[n] >= mx - 2.0f && g4o_cap(lg[n]) == cm) {
        best = n;
        break;
      }
  }
  info->vmax = mx;
  info->G = best;
  free(xe);
  free(xo);
  free(gs);
  free(s);
  free(U);
  free(L);
}

/* ------------------------------------------------------------------------ */
/* split-KV attention                                                       */
/* ------------------------------------------------------------------------ */

/* E:740 attn_allowed */
static inline int allowed(const int* pos, const int* lo, const int* sl, const int* sh, int m, int p) {
  return p >= lo[m] && p <= pos[m] && !(p >= sl[m] && p <= sh[m]);
}

/* E:743-877 attn_task for split t of T and E:1019-1059 attn_merge (output rounded to bf16).
 * q rows [M][nh*hd] (ldq), out rows [M][nh*hd] (ldo).  Per (m, h):
 *   pass 1: score_p = hsum(s0 + s1), s0/s1 8-lane FMA chains over hd in steps of 16;
 *           running max per split;
 *   pass 2: w_p = exp8(score_p - max) in position order, l += w, o = fma(w, v_p, o);
 *   merge : M0 = max over splits with l > 0, sc_t = expf(max_t - M0) (libm),
 *           l = sum (double) l_t sc_t, out = r16((sum_t fma(o_t, sc_t)) * (float)(1/l)).
 * part_m/part_l (optional, [T][M][nh]) receive the per-split max and sum. */
void g4o_attn_splitkv(const uint16_t* Kc, const uint16_t* Vc, int hd, int nh, int M,
                      const float* q, int ldq, const int* pos, const int* lo, const int* skip_lo,
                      const int* skip_hi, int kmin, int kmax, int T, float* out, int ldo,
                      float* part_m, float* part_l) {
  const int len = kmax - kmin + 1;
  float* AO = (float*)calloc((size_t)T * M * nh * hd, sizeof(float));
  float* AM = (float*)malloc(sizeof(float) * (size_t)T * M * nh);
  float* AL = (float*)malloc(sizeof(float) * (size_t)T * M * nh);
  float* sc = (float*)malloc(sizeof(float) * (size_t)(len > 0 ? len : 1) * nh);
  float* kf = (float*)malloc(sizeof(float) * hd);
  for (int t = 0; t < T; ++t) {
    const int c0 = kmin + (int)((long)t * len / T), c1 = kmin + (int)((long)(t + 1) * len / T);
    for (int m = 0; m < M; ++m) {
      for (int h = 0; h < nh; ++h) {
        const float* qh = q + (size_t)m * ldq + (size_t)h * hd;
        float mx = -1e30f;
        for (int p = c0; p < c1; ++p) {
          if (!allowed(pos, lo, skip_lo, skip_hi, m, p)) continue;
          for (int i = 0; i < hd; ++i) kf[i] = g4o_bf2f(Kc[(size_t)p * hd + i]);
          float s0[8] = {0}, s1[8] = {0};
          for (int i = 0; i < hd; i += 16)
            for (int l = 0; l < 8; ++l) {
              s0[l] = fmaf(qh[i + l], kf[i + l], s0[l]);
              s1[l] = fmaf(qh[i + 8 + l], kf[i + 8 + l], s1[l]);
            }
          float v[8];
          for (int l = 0; l < 8; ++l) v[l] = s0[l] + s1[l];
          float s = hsum8(v);
          sc[(size_t)(p - c0) * nh + h] = s;
          mx = (mx < s) ? s : mx;
        }
        float l = 0.f;
        float* o = AO + (((size_t)t * M + m) * nh + h) * hd;
        for (int p = c0; p < c1; ++p) {
          if (!allowed(pos, lo, skip_lo, skip_hi, m, p)) continue;
          float w = g4o_exp8(sc[(size_t)(p - c0) * nh + h] - mx);
          l = l + w;
          for (int i = 0; i < hd; ++i) o[i] = fmaf(w, g4o_bf2f(Vc[(size_t)p * hd + i]), o[i]);
        }
        AM[((size_t)t * M + m) * nh + h] = mx;
        AL[((size_t)t * M + m) * nh + h] = (lo[m] > pos[m]) ? 0.0f : l;
      }
    }
  }
  for (int m = 0; m < M; ++m)
    for (int h = 0; h < nh; ++h) {
      float M0 = -1e30f;
      for (int t = 0; t < T; ++t) {
        size_t k = ((size_t)t * M + m) * nh + h;
        if (AL[k] > 0) M0 = (M0 < AM[k]) ? AM[k] : M0;
      }
      double l = 0;
      float scs[64];
      int act[64], na = 0;
      for (int t = 0; t < T; ++t) {
        size_t k = ((size_t)t * M + m) * nh + h;
        if (!(AL[k] > 0)) continue;
        float s = expf(AM[k] - M0);
        l = fma((double)AL[k], (double)s, l);
        scs[na] = s;
        act[na] = t;
        ++na;
      }
      const float inv = (float)(1.0 / l);
      float* oo = out + (size_t)m * ldo + (size_t)h * hd;
      for (int i = 0; i < hd; ++i) {
        float acc = 0.f;
        for (int k = 0; k < na; ++k)
          acc = fmaf(AO[(((size_t)act[k] * M + m) * nh + h) * hd + i], scs[k], acc);
        oo[i] = g4o_r16(acc * inv);
      }
    }
  if (part_m) memcpy(part_m, AM, sizeof(float) * (size_t)T * M * nh);
  if (part_l) memcpy(part_l, AL, sizeof(float) * (size_t)T * M * nh);
  free(AO);
  free(AM);
  free(AL);
  free(sc);
  free(kf);
}

/* ------------------------------------------------------------------------ */
/* seeded input generators (formulas in g4_rng.h)                           */
/* ------------------------------------------------------------------------ */
uint64_t g4o_stream(uint64_t seed, uint64_t tag) { return g4r_stream(seed, tag); }
void g4o_gen_normal_f32(uint64_t seed, int64_t n, float scale, float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = scale * g4r_normal(seed, (uint64_t)i);
}
void g4o_gen_normal_bf16(uint64_t seed, int64_t n, float scale, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = g4o_f2bf(scale * g4r_normal(seed, (uint64_t)i));
}
void g4o_gen_bytes(uint64_t seed, int64_t n, uint8_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = (uint8_t)((g4r_hash(seed, (uint64_t)i) >> 24) & 0xFF);
}
void g4o_gen_scales(uint64_t seed, int64_t n, float lo, float span, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = g4o_f2bf(lo + span * g4r_unif(seed, (uint64_t)i));
}
void g4o_gen_ints(uint64_t seed, int64_t n, int32_t lo, int32_t hi, int32_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) out[i] = g4r_int(seed, (uint64_t)i, lo, hi);
}

/* ------------------------------------------------------------------------ */
/* prefill attention                                                         */
/* ------------------------------------------------------------------------ */

/* E:1063-1083 attn_tile, row by row: a row's result depends only on its own range
 * [lo, pos], not on the tile of QB rows it shares K/V loads with.  Per (m, h):
 *   s_p = hsum(s0 + s1) (s0/s1 8-lane FMA chains over hd in steps of 16), mx = max_p s_p;
 *   in position order: w = exp8(s_p - mx), den += w, O = fma(w, v_p, O);
 *   out = r16(O * (1 / den)). */
void g4o_attn_tile(const uint16_t* Kc, const uint16_t* Vc, int hd, int nh, int M, const float* q, int ldq,
                   const int* pos, const int* lo, float* out, int ldo) {
  float* kf = (float*)malloc(sizeof(float) * hd);
  float* O = (float*)malloc(sizeof(float) * hd);
  for (int m = 0; m < M; ++m) {
    const int len = pos[m] - lo[m] + 1;
    float* sc = (float*)malloc(sizeof(float) * (size_t)(len > 0 ? len : 1));
    for (int h = 0; h < nh; ++h) {
      const float* qh = q + (size_t)m * ldq + (size_t)h * hd;
      float mx = -1e30f;
      for (int p = lo[m]; p <= pos[m]; ++p) {
        for (int i = 0; i < hd; ++i) kf[i] = g4o_bf2f(Kc[(size_t)p * hd + i]);
        float s0[8] = {0}, s1[8] = {0}, v[8];
        for (int i = 0; i < hd; i += 16)
          for (int l = 0; l < 8; ++l) {
            s0[l] = fmaf(qh[i + l], kf[i + l], s0[l]);
            s1[l] = fmaf(qh[i + 8 + l], kf[i + 8 + l], s1[l]);
          }
        for (int l = 0; l < 8; ++l) v[l] = s0[l] + s1[l];
        const float s = hsum8(v);
        sc[p - lo[m]] = s;
        mx = (mx < s) ? s : mx;
      }
      float den = 0.f;
      for (int i = 0; i < hd; ++i) O[i] = 0.f;
      for (int p = lo[m]; p <= pos[m]; ++p) {
        const float w = g4o_exp8(sc[p - lo[m]] - mx);
        den += w;
        for (int i = 0; i < hd; ++i) O[i] = fmaf(w, g4o_bf2f(Vc[(size_t)p * hd + i]), O[i]);
      }
      const float inv = 1.0f / den;
      float* oo = out + (size_t)m * ldo + (size_t)h * hd;
      for (int i = 0; i < hd; ++i) oo[i] = g4o_r16(O[i] * inv);
    }
    free(sc);
  }
  free(kf);
  free(O);
}

/* E:1338-1349 run_mh (no sibling row), per (m, h):
 *   d_p = hsum(sv) (one 8-lane FMA chain over hd in steps of 8), mx = max_p d_p;
 *   e_p = expf(d_p - mx) (libm), den = sum_p e_p in position order;
 *   in position order: o = fma(e_p / den, v_p, o);  out = r16(o). */
void g4o_attn_mh(const uint16_t* Kc, const uint16_t* Vc, int hd, int nh, int M, const float* q, int ldq,
                 const int* pos, const int* lo, const int* skip_lo, const int* skip_hi, float* out, int ldo) {
  for (int m = 0; m < M; ++m) {
    const int len = pos[m] - lo[m] + 1;
    /* E:1345 valid(p): the sibling row skips the chain rows between row 0 and itself */
    const int s0 = skip_lo ? skip_lo[m] : 1, s1 = skip_hi ? skip_hi[m] : 0;
#define MH_VALID(p) (!((p) >= s0 && (p) <= s1))
    float* sc = (float*)malloc(sizeof(float) * (size_t)(len > 0 ? len : 1));
    for (int h = 0; h < nh; ++h) {
      const float* qh = q + (size_t)m * ldq + (size_t)h * hd;
      float mx = -1e30f;
      for (int p = lo[m]; p <= pos[m]; ++p) {
        if (!MH_VALID(p)) continue;
        float sv[8] = {0};
        for (int i = 0; i < hd; i += 8)
          for (int l = 0; l < 8; ++l) sv[l] = fmaf(qh[i + l], g4o_bf2f(Kc[(size_t)p * hd + i + l]), sv[l]);
        const float d = hsum8(sv);
        sc[p - lo[m]] = d;
        mx = (mx < d) ? d : mx;
      }
      float den = 0.f;
      for (int p = lo[m]; p <= pos[m]; ++p) {
        if (!MH_VALID(p)) continue;
        sc[p - lo[m]] = expf(sc[p - lo[m]] - mx);
        den += sc[p - lo[m]];
      }
      float* oo = out + (size_t)m * ldo + (size_t)h * hd;
      for (int i = 0; i < hd; ++i) oo[i] = 0.f;
      for (int p = lo[m]; p <= pos[m]; ++p) {
        if (!MH_VALID(p)) continue;
        const float wgt = sc[p - lo[m]] / den;
        for (int i = 0; i < hd; ++i) oo[i] = fmaf(wgt, g4o_bf2f(Vc[(size_t)p * hd + i]), oo[i]);
      }
      for (int i = 0; i < hd; ++i) oo[i] = g4o_r16(oo[i]);
    }
#undef MH_VALID
    free(sc);
  }
}
