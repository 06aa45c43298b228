// g4v_layer.hip -- split-KV attention, RMSNorm row kernels, q/k norm + RoPE + KV write,
// branch selection and acceptance for one verify pass on gfx950.
//
// References (E = engine/gemma4_engine.cpp): embedding E:1262-1267; q/k/v norm, RoPE and KV
// write E:1307-1324; attn_task E:743-877; attn_merge E:1019-1059; residual/norm blocks
// E:1358-1361, E:1375-1404; lazy head + acceptance E:1453-1488, E:1647-1661.
#include "g4v_layer.h"

namespace g4v {

__constant__ uint64_t c_expf_tab[32] = G4V_EXPF_TABLE;

// E:326-343 ss_avx2: lane t (0..15) accumulates x[16 s + t]^2 in double over steps s;
// s[k][l] = lane 4k + l; a[l] = (s[0][l]+s[1][l])+(s[2][l]+s[3][l]); ss = (a0+a2)+(a1+a3).
// x is in LDS; red16 is LDS scratch; every thread returns ss.
__device__ double block_sumsq(const float* x, int n, double* red16) {
  if (threadIdx.x < 16) {
    double s = 0;
    for (int i = threadIdx.x; i < n; i += 16) {
      const double d = (double)x[i];
      s = fma(d, d, s);
    }
    red16[threadIdx.x] = s;
  }
  __syncthreads();
  double a[4];
  for (int l = 0; l < 4; ++l) a[l] = (red16[l] + red16[4 + l]) + (red16[8 + l] + red16[12 + l]);
  const double ss = (a[0] + a[2]) + (a[1] + a[3]);
  __syncthreads();
  return ss;
}

// E:345: r = 1 / sqrtf((float)(ss / n) + 1e-6)
__device__ __forceinline__ float rms_inv(double ss, int n) { return 1.0f / sqrtf((float)(ss / n) + 1e-6f); }

constexpr int ROW_THREADS = 256;

// E:1262-1267: x = rbf8(E[tok] * sqrt(H)); xa = (x * r) * in_ln
__global__ __launch_bounds__(ROW_THREADS) void k_embed(const uint16_t* __restrict__ E, const StepDev* sp,
                                                       const float* __restrict__ in_ln, float sqh,
                                                       float* __restrict__ x, float* __restrict__ xa) {
  __shared__ float xs[H];
  __shared__ double red[16];
  const int m = blockIdx.x;
  const int tok = sp->toks[m];
  for (int i = threadIdx.x; i < H; i += ROW_THREADS) {
    const float v = r16(bf2f(E[(size_t)tok * H + i]) * sqh);
    xs[i] = v;
    x[(size_t)m * H + i] = v;
  }
  __syncthreads();
  const float r = rms_inv(block_sumsq(xs, H, red), H);
  for (int i = threadIdx.x; i < H; i += ROW_THREADS) xa[(size_t)m * H + i] = (xs[i] * r) * in_ln[i];
}

// E:1358-1361: o = r16(o); tmp = rms(o, post_attn); x = r16(x + r16(tmp)); xa = r16(rms(x, pre_ff))
__global__ __launch_bounds__(ROW_THREADS) void k_post_attn(const float* __restrict__ o, float* __restrict__ x,
                                                           float* __restrict__ xa, LayerNorms ln) {
  __shared__ float os[H], xs[H];
  __shared__ double red[16];
  const int m = blockIdx.x;
  for (int i = threadIdx.x; i < H; i += ROW_THREADS) os[i] = r16(o[(size_t)m * H + i]);
  __syncthreads();
  const float r1 = rms_inv(block_sumsq(os, H, red), H);
  for (int i = threadIdx.x; i < H; i += ROW_THREADS) {
    const float tmp = (os[i] * r1) * ln.post_attn[i];
    const float v = r16(x[(size_t)m * H + i] + r16(tmp));
    xs[i] = v;
    x[(size_t)m * H + i] = v;
  }
  __syncthreads();
  const float r2 = rms_inv(block_sumsq(xs, H, red), H);
  for (int i = threadIdx.x; i < H; i += ROW_THREADS) xa[(size_t)m * H + i] = r16((xs[i] * r2) * ln.pre_ff[i]);
}

// E:1375-1378 and E:1390-1404 with a zero per-layer-embedding branch:
// o = r16(o); tmp = rms(o, post_ff); x = r16(x + r16(tmp)); x = r16(x * scalar);
// then xa = rms(x, next in_ln) or, after the last layer, h = r16(rms(x, fnorm)), hn = |h|.
__global__ __launch_bounds__(ROW_THREADS) void k_post_ff(const float* __restrict__ o, float* __restrict__ x,
                                                         float* __restrict__ xa, LayerNorms ln,
                                                         const float* __restrict__ next_in_ln,
                                                         const float* __restrict__ fnorm, float* __restrict__ h,
                                                         float* __restrict__ hn) {
  __shared__ float os[H], xs[H];
  __shared__ double red[16];
  const int m = blockIdx.x;
  for (int i = threadIdx.x; i < H; i += ROW_THREADS) os[i] = r16(o[(size_t)m * H + i]);
  __syncthreads();
  const float r1 = rms_inv(block_sumsq(os, H, red), H);
  for (int i = threadIdx.x; i < H; i += ROW_THREADS) {
    const float tmp = (os[i] * r1) * ln.post_ff[i];
    float v = r16(x[(size_t)m * H + i] + r16(tmp));
    v = r16(v * ln.scalar);
    xs[i] = v;
    x[(size_t)m * H + i] = v;
  }
  __syncthreads();
  const float r2 = rms_inv(block_sumsq(xs, H, red), H);
  if (next_in_ln) {
    for (int i = threadIdx.x; i < H; i += ROW_THREADS) xa[(size_t)m * H + i] = (xs[i] * r2) * next_in_ln[i];
  } else {
    for (int i = threadIdx.x; i < H; i += ROW_THREADS) {
      const float v = r16((xs[i] * r2) * fnorm[i]);
      os[i] = v;
      h[(size_t)m * H + i] = v;
    }
    __syncthreads();
    const double ss = block_sumsq(os, H, red);
    if (threadIdx.x == 0) hn[m] = (float)sqrt(ss);  // E:1417
  }
}

// E:1307-1324: per row m, blocks h < 8 normalise + rotate query head h (E:1312), block 8
// normalises + rotates k (E:1316) and normalises v (E:1317), then writes both to the cache slot.
__global__ __launch_bounds__(HD) void k_qk_rope(float* __restrict__ q, const float* __restrict__ k,
                                                const float* __restrict__ v, int ldq, const StepDev* sp,
                                                LayerNorms ln, const float* __restrict__ cs,
                                                const float* __restrict__ sn, uint16_t* __restrict__ KC,
                                                uint16_t* __restrict__ VC) {
  __shared__ float ys[HD];
  __shared__ double red[16];
  const int m = blockIdx.x, hh = blockIdx.y, i = threadIdx.x;
  const int rp = sp->rope[m], slot = sp->pos0 + m;
  const float* src = hh < NQ ? q + (size_t)m * ldq + hh * HD : k + (size_t)m * HD;
  const float* w = hh < NQ ? ln.qn : ln.kn;
  ys[i] = src[i];
  __syncthreads();
  const float r = rms_inv(block_sumsq(ys, HD, red), HD);
  const float y = r16((ys[i] * r) * w[i]);
  __syncthreads();
  ys[i] = y;
  __syncthreads();
  float outv;
  if (i < HD / 2) {  // E:394-402 NeoX halves
    const float u = ys[i], ww = ys[i + HD / 2], c = cs[(size_t)rp * (HD / 2) + i], s = sn[(size_t)rp * (HD / 2) + i];
    outv = fmaf(u, c, -(ww * s));
  } else {
    const int jj = i - HD / 2;
    const float u = ys[jj], ww = ys[i], c = cs[(size_t)rp * (HD / 2) + jj], s = sn[(size_t)rp * (HD / 2) + jj];
    outv = fmaf(ww, c, u * s);
  }
  if (hh < NQ) {
    q[(size_t)m * ldq + hh * HD + i] = outv;
  } else {
    KC[(size_t)slot * HD + i] = f2bf(outv);
    __syncthreads();
    ys[i] = v[(size_t)m * HD + i];
    __syncthreads();
    const float rv = rms_inv(block_sumsq(ys, HD, red), HD);
    VC[(size_t)slot * HD + i] = f2bf(r16(ys[i] * rv));
  }
}

// ---------------------------------------------------------------------------------------
// split-KV attention (E:743-877) and merge (E:1019-1059)
// ---------------------------------------------------------------------------------------
constexpr int ATT_THREADS = 256;
constexpr int ATT_TILE = 32;     // K rows per tile, 8 lanes per row
constexpr int ATT_SCAP = 8448;   // LDS floats for the [M][P] scores of one split

__device__ __forceinline__ bool att_allowed(const AttnGeom& g, int m, int p) {
  return p >= g.lo[m] && p <= g.pos[m] && !(p >= g.skip_lo[m] && p <= g.skip_hi[m]);
}

// E:1325-1326 geometry of a verify pass
__device__ void geom_from_step(const StepDev* sp, int sliding, int T, AttnGeom& g) {
  g.M = sp->M;
  g.T = T;
  g.kmax = sp->pos0 + sp->M - 1;
  g.kmin = g.kmax;
  for (int r = 0; r < sp->M; ++r) {
    g.pos[r] = sp->pos0 + r;
    g.lo[r] = sliding ? max(0, sp->rope[r] - 511) : 0;
    g.skip_lo[r] = sp->skip_lo[r];
    g.skip_hi[r] = sp->skip_hi[r];
    g.kmin = min(g.kmin, g.lo[r]);
  }
}

struct AttnPtrs {
  const uint16_t* KC;
  const uint16_t* VC;
  const float* q;
  int ldq;
  float* po;  // [T][M][NQ][HD]
  float* pm;  // [T][M][NQ]
  float* pl;  // [T][M][NQ]
  float* out; // [M][ldo]
  int ldo;
};

// one block per (split t, head h)
template <bool STEP>
__global__ __launch_bounds__(ATT_THREADS) void k_attn_split(AttnPtrs P, AttnGeom gin, const StepDev* sp, int sliding,
                                                            int T) {
  __shared__ AttnGeom g;
  __shared__ float qs[MAXM][HD];
  __shared__ uint16_t kt[ATT_TILE][HD + 16];
  __shared__ float sw[ATT_SCAP];
  __shared__ float wmax[ATT_THREADS / 64][MAXM];
  __shared__ float smax[MAXM], ssum[MAXM];
  const int t = blockIdx.x, h = blockIdx.y;
  if (threadIdx.x == 0) {
    if (STEP) geom_from_step(sp, sliding, T, g);
    else g = gin;
  }
  __syncthreads();
  const int M = g.M;
  const int len = g.kmax - g.kmin + 1;
  const int c0 = g.kmin + (int)((long)t * len / T), c1 = g.kmin + (int)((long)(t + 1) * len / T);
  const int PP = c1 - c0;
  for (int idx = threadIdx.x; idx < M * HD; idx += ATT_THREADS) {
    const int m = idx / HD, i = idx % HD;
    qs[m][i] = P.q[(size_t)m * P.ldq + h * HD + i];
  }
  const int ps = threadIdx.x >> 3, l = threadIdx.x & 7;
  float mymax[MAXM];
#pragma unroll
  for (int m = 0; m < MAXM; ++m) mymax[m] = -1e30f;
  // pass 1: scores; lane l of a position holds the two 8-lane chains (E:770-779)
  for (int pb = c0; pb < c1; pb += ATT_TILE) {
    __syncthreads();
    for (int u = threadIdx.x; u < ATT_TILE * (HD / 8); u += ATT_THREADS) {
      const int rr = u / (HD / 8), cc = u % (HD / 8), p = pb + rr;
      uint4 val = make_uint4(0, 0, 0, 0);
      if (p < c1) val = reinterpret_cast<const uint4*>(P.KC + (size_t)p * HD)[cc];
      uint4* dst = reinterpret_cast<uint4*>(&kt[rr][cc * 8]);
      *dst = val;
    }
    __syncthreads();
    const int p = pb + ps;
    if (p < c1) {
      for (int m = 0; m < M; ++m) {
        if (!att_allowed(g, m, p)) continue;
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int tt = 0; tt < HD / 16; ++tt) {
          s0 = fmaf(qs[m][16 * tt + l], bf2f(kt[ps][16 * tt + l]), s0);
          s1 = fmaf(qs[m][16 * tt + 8 + l], bf2f(kt[ps][16 * tt + 8 + l]), s1);
        }
        float v = s0 + s1;
        v = v + __shfl_xor(v, 4, 8);
        v = v + __shfl_xor(v, 1, 8);
        v = v + __shfl_xor(v, 2, 8);
        if (l == 0) {
          sw[m * PP + (p - c0)] = v;
          mymax[m] = (mymax[m] < v) ? v : mymax[m];
        }
      }
    }
  }
  // running max of the split (order free)
#pragma unroll
  for (int m = 0; m < MAXM; ++m) {
    float v = mymax[m];
    for (int s = 8; s < 64; s <<= 1) v = fmaxf(v, __shfl_xor(v, s, 64));
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6][m] = v;
  }
  __syncthreads();
  if (threadIdx.x < MAXM) {
    float v = -1e30f;
    for (int w = 0; w < ATT_THREADS / 64; ++w) v = (v < wmax[w][threadIdx.x]) ? wmax[w][threadIdx.x] : v;
    smax[threadIdx.x] = v;
  }
  __syncthreads();
  // pass 2a: weights exp8(score - max) (E:820)
  for (int idx = threadIdx.x; idx < M * PP; idx += ATT_THREADS) {
    const int m = idx / PP, pp = idx % PP;
    if (att_allowed(g, m, c0 + pp)) sw[idx] = exp8(sw[idx] - smax[m]);
  }
  __syncthreads();
  // pass 2b: l = sum of weights in position order; o_i = fma chain over positions (E:821-875)
  if (threadIdx.x < M) {
    const int m = threadIdx.x;
    float lsum = 0.f;
    for (int pp = 0; pp < PP; ++pp)
      if (att_allowed(g, m, c0 + pp)) lsum = lsum + sw[m * PP + pp];
    ssum[m] = (g.lo[m] > g.pos[m]) ? 0.0f : lsum;
  }
  const int i = threadIdx.x;
  float o[MAXM];
#pragma unroll
  for (int m = 0; m < MAXM; ++m) o[m] = 0.f;
  for (int pp = 0; pp < PP; ++pp) {
    const float vv = bf2f(P.VC[(size_t)(c0 + pp) * HD + i]);
#pragma unroll
    for (int m = 0; m < MAXM; ++m)
      if (m < M && att_allowed(g, m, c0 + pp)) o[m] = fmaf(sw[m * PP + pp], vv, o[m]);
  }
  __syncthreads();
  for (int m = 0; m < M; ++m) P.po[(((size_t)t * M + m) * NQ + h) * HD + i] = o[m];
  if (threadIdx.x < M) {
    P.pm[((size_t)t * M + threadIdx.x) * NQ + h] = smax[threadIdx.x];
    P.pl[((size_t)t * M + threadIdx.x) * NQ + h] = ssum[threadIdx.x];
  }
}

// E:1019-1059: M0 = max over splits with l > 0; sc = expf(max_t - M0); l = sum (double) l_t sc;
// out = r16((fma chain over splits of o_t sc) * (float)(1/l)).  One block per (m, h).
__global__ __launch_bounds__(HD) void k_attn_merge(AttnPtrs P, int M, int T) {
  const int m = blockIdx.x, h = blockIdx.y, i = threadIdx.x;
  float M0 = -1e30f;
  for (int t = 0; t < T; ++t) {
    const size_t k = ((size_t)t * M + m) * NQ + h;
    if (P.pl[k] > 0) M0 = (M0 < P.pm[k]) ? P.pm[k] : M0;
  }
  double l = 0;
  float scs[MAXT];
  int act[MAXT], na = 0;
  for (int t = 0; t < T; ++t) {
    const size_t k = ((size_t)t * M + m) * NQ + h;
    if (!(P.pl[k] > 0)) continue;
    const float sc = libm_expf_neg(P.pm[k] - M0, c_expf_tab);
    l = fma((double)P.pl[k], (double)sc, l);
    scs[na] = sc;
    act[na] = t;
    ++na;
  }
  const float inv = (float)(1.0 / l);
  float acc = 0.f;
  for (int kk = 0; kk < na; ++kk) acc = fmaf(P.po[(((size_t)act[kk] * M + m) * NQ + h) * HD + i], scs[kk], acc);
  P.out[(size_t)m * P.ldo + h * HD + i] = r16(acc * inv);
}

// read M from the step block for the graph-captured path
__global__ __launch_bounds__(HD) void k_attn_merge_step(AttnPtrs P, const StepDev* sp, int T) {
  if ((int)blockIdx.x >= sp->M) return;
  // same body with M from the step parameters
  const int M = sp->M, m = blockIdx.x, h = blockIdx.y, i = threadIdx.x;
  float M0 = -1e30f;
  for (int t = 0; t < T; ++t) {
    const size_t k = ((size_t)t * M + m) * NQ + h;
    if (P.pl[k] > 0) M0 = (M0 < P.pm[k]) ? P.pm[k] : M0;
  }
  double l = 0;
  float scs[MAXT];
  int act[MAXT], na = 0;
  for (int t = 0; t < T; ++t) {
    const size_t k = ((size_t)t * M + m) * NQ + h;
    if (!(P.pl[k] > 0)) continue;
    const float sc = libm_expf_neg(P.pm[k] - M0, c_expf_tab);
    l = fma((double)P.pl[k], (double)sc, l);
    scs[na] = sc;
    act[na] = t;
    ++na;
  }
  const float inv = (float)(1.0 / l);
  float acc = 0.f;
  for (int kk = 0; kk < na; ++kk) acc = fmaf(P.po[(((size_t)act[kk] * M + m) * NQ + h) * HD + i], scs[kk], acc);
  P.out[(size_t)m * P.ldo + h * HD + i] = r16(acc * inv);
}

// ---------------------------------------------------------------------------------------
// branch choice between the two head passes, acceptance and KV compaction
// ---------------------------------------------------------------------------------------
// E:1477-1484 generalised: after row 0, walk chain a when G[0] == toks[1], otherwise branch b
// when G[0] == toks[b1]; the second head pass evaluates that branch's rows.
__global__ void k_branch(const StepDev* sp, const int* best1, const float* __restrict__ h,
                         const float* __restrict__ hn, float* __restrict__ h2, float* __restrict__ hn2,
                         VerifyResultDev* res) {
  __shared__ int first, cnt;
  if (threadIdx.x == 0) {
    const int G0 = best1[0];
    first = 0;
    cnt = 0;
    if (sp->na >= 1 && sp->toks[1] == G0) {
      first = 1;
      cnt = sp->na;
    } else if (sp->nb >= 1 && sp->toks[sp->na + 1] == G0) {
      first = sp->na + 1;
      cnt = sp->nb;
    }
    res->hcount = cnt;
    for (int r = 0; r < MAXM; ++r) res->hrows[r] = r < cnt ? first + r : -1;
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < cnt * H; idx += blockDim.x) h2[idx] = h[(size_t)first * H + idx];
  if (threadIdx.x < cnt) hn2[threadIdx.x] = hn[first + threadIdx.x];
}

// E:1647-1661: nacc = longest accepted prefix along the evaluated branch; commit G on the path
__global__ void k_accept(const StepDev* sp, const int* best1, const int* best2, const int* cnt1, const int* cnt2,
                         VerifyResultDev* res) {
  if (threadIdx.x != 0) return;
  for (int r = 0; r < MAXM; ++r) {
    res->G[r] = -1;
    res->fallback[r] = 0;
    res->nsurv[r] = 0;
  }
  res->G[0] = best1[0];
  res->nsurv[0] = cnt1[0];
  res->fallback[0] = cnt1[0] > HEAD_LIMIT;
  int path[MAXM], np = 1;
  path[0] = 0;
  const int cnt = res->hcount;
  int prevG = best1[0];
  for (int r = 0; r < cnt; ++r) {
    const int row = res->hrows[r];
    if (prevG != sp->toks[row]) break;
    res->G[row] = best2[r];
    res->nsurv[row] = cnt2[r];
    res->fallback[row] = cnt2[r] > HEAD_LIMIT;
    prevG = best2[r];
    path[np++] = row;
  }
  res->nacc = np - 1;
  res->branch = (np > 1 && path[1] > sp->na) ? 1 : 0;
  res->ncommit = np;
  for (int r = 0; r < MAXM; ++r) res->commit[r] = r < np ? res->G[path[r]] : -1;
  for (int r = 0; r < MAXM; ++r) res->hrows[r] = r < np ? path[r] : -1;  // the committed path
}

// E:1651: branch b commits by moving its cache rows to the positions after row 0 (every layer)
__global__ void k_kv_compact(const StepDev* sp, const VerifyResultDev* res, uint16_t* KC, uint16_t* VC, int ctxcap) {
  if (res->branch != 1) return;
  const int l = blockIdx.x, i = threadIdx.x;
  for (int r = 1; r < res->ncommit; ++r) {
    const size_t src = ((size_t)l * ctxcap + sp->pos0 + res->hrows[r]) * HD + i;
    const size_t dst = ((size_t)l * ctxcap + sp->pos0 + r) * HD + i;
    KC[dst] = KC[src];
    VC[dst] = VC[src];
  }
}

// ---------------------------------------------------------------------------------------
// synthetic weights
// ---------------------------------------------------------------------------------------
__global__ void k_gen_bf16_normal(uint16_t* out, size_t n, uint64_t seed, float scale) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    out[i] = f2bf(scale * rng_normal(seed, i));
}
__global__ void k_gen_w4(uint8_t* w, uint16_t* s, size_t nb, size_t ns, uint64_t sw, uint64_t ss) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < nb; i += (size_t)gridDim.x * blockDim.x)
    w[i] = (uint8_t)((rng_hash(sw, i) >> 24) & 0xFF);
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < ns; i += (size_t)gridDim.x * blockDim.x)
    s[i] = f2bf(0.005f + 0.015f * rng_unif(ss, i));
}

// ---------------------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------------------
void launch_embed(const uint16_t* E, const StepDev* sp, const float* in_ln, float sqh, float* x, float* xa, int M,
                  hipStream_t st) {
  hipLaunchKernelGGL(k_embed, dim3(M), dim3(ROW_THREADS), 0, st, E, sp, in_ln, sqh, x, xa);
}
void launch_qk_rope(float* q, const float* k, const float* v, int ldq, const StepDev* sp, const LayerNorms& ln,
                    const float* cs, const float* sn, uint16_t* KC, uint16_t* VC, int M, hipStream_t st) {
  hipLaunchKernelGGL(k_qk_rope, dim3(M, NQ + 1), dim3(HD), 0, st, q, k, v, ldq, sp, ln, cs, sn, KC, VC);
}
void launch_attn(const uint16_t* KC, const uint16_t* VC, const float* q, const StepDev* sp, int sliding, int T,
                 int ctxcap, float* po, float* pm, float* pl, float* att, int M, hipStream_t st) {
  (void)ctxcap;
  AttnPtrs P{KC, VC, q, NQ * HD, po, pm, pl, att, NQ * HD};
  AttnGeom g{};
  hipLaunchKernelGGL(k_attn_split<true>, dim3(T, NQ), dim3(ATT_THREADS), 0, st, P, g, sp, sliding, T);
  hipLaunchKernelGGL(k_attn_merge_step, dim3(M, NQ), dim3(HD), 0, st, P, sp, T);
}
void launch_attn_geom(const uint16_t* KC, const uint16_t* VC, const float* q, int ldq, const AttnGeom& g,
                      float* po, float* pm, float* pl, float* out, int ldo, hipStream_t st) {
  AttnPtrs P{KC, VC, q, ldq, po, pm, pl, out, ldo};
  hipLaunchKernelGGL(k_attn_split<false>, dim3(g.T, NQ), dim3(ATT_THREADS), 0, st, P, g, (const StepDev*)nullptr, 0,
                     g.T);
  hipLaunchKernelGGL(k_attn_merge, dim3(g.M, NQ), dim3(HD), 0, st, P, g.M, g.T);
}
void launch_post_attn(const float* o, float* x, float* xa, const LayerNorms& ln, int M, hipStream_t st) {
  hipLaunchKernelGGL(k_post_attn, dim3(M), dim3(ROW_THREADS), 0, st, o, x, xa, ln);
}
void launch_post_ff(const float* o, float* x, float* xa, const LayerNorms& ln, const float* next_in_ln,
                    const float* fnorm, float* h, float* hn, int M, hipStream_t st) {
  hipLaunchKernelGGL(k_post_ff, dim3(M), dim3(ROW_THREADS), 0, st, o, x, xa, ln, next_in_ln, fnorm, h, hn);
}
void launch_branch(const StepDev* sp, const int* best1, const float* h, const float* hn, float* h2, float* hn2,
                   VerifyResultDev* res, hipStream_t st) {
  hipLaunchKernelGGL(k_branch, dim3(1), dim3(256), 0, st, sp, best1, h, hn, h2, hn2, res);
}
void launch_accept(const StepDev* sp, const int* best1, const int* best2, const int* cnt1, const int* cnt2,
                   VerifyResultDev* res, uint16_t* KC, uint16_t* VC, int NL, int ctxcap, hipStream_t st) {
  hipLaunchKernelGGL(k_accept, dim3(1), dim3(64), 0, st, sp, best1, best2, cnt1, cnt2, res);
  hipLaunchKernelGGL(k_kv_compact, dim3(NL), dim3(HD), 0, st, sp, res, KC, VC, ctxcap);
}
void launch_gen_bf16_normal(uint16_t* out, size_t n, uint64_t seed, float scale, hipStream_t st) {
  size_t g = (n + 255) / 256;
  hipLaunchKernelGGL(k_gen_bf16_normal, dim3(g > 65536 ? 65536 : (unsigned)g), dim3(256), 0, st, out, n, seed, scale);
}
void launch_gen_w4(uint8_t* w, uint16_t* s, size_t nbytes, size_t nscales, uint64_t sw, uint64_t ss,
                   hipStream_t st) {
  size_t g = (nbytes + 255) / 256;
  hipLaunchKernelGGL(k_gen_w4, dim3(g > 65536 ? 65536 : (unsigned)g), dim3(256), 0, st, w, s, nbytes, nscales, sw, ss);
}

}  // namespace g4v
