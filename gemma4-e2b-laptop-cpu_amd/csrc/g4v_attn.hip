// g4v_attn.hip -- split-KV attention over the draft rows (E:743-877) and the exact
// log-sum-exp merge of the splits (E:1019-1059), gfx950.  E = engine/gemma4_engine.cpp.
//
// Split t covers keys [kmin + t*len/T, kmin + (t+1)*len/T) exactly as the reference's
// worker t does, and every per-(row, head) value is produced in the reference's fp32 order:
//   score_p = hsum8(s0 + s1), s0/s1 two 8-lane FMA chains over the head dim in steps of 16;
//   w_p = exp8(score_p - max), l = sum of w_p in position order, o_i = fma chain over p;
//   merge: sc_t = libm expf(max_t - M0), l = sum_t (double) l_t sc_t,
//          out = r16((fma chain over splits of o_t sc_t) * (float)(1 / l)).
// One block serves (split t, row m, 4 heads): the block's K/V rows are staged through LDS
// tile by tile (the next tile is fetched into registers while the current one is used) and
// shared by the 4 heads.
#include "g4v_layer.h"

namespace g4v {

__constant__ uint64_t c_expf_tab[32] = G4V_EXPF_TABLE;

constexpr int ATT_THREADS = 256;
constexpr int ATT_TILE = 32;  // key rows per tile: 8 lanes per row, 32 rows
constexpr int ATT_HB = 4;     // heads per block
constexpr int ATT_PMAX = 1040;  // positions per split held in LDS

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

// 32 key rows x 256 bf16 = 1024 16-byte chunks: 4 per thread
__device__ __forceinline__ void tile_fetch(const uint16_t* base, int p0, int c1, uint4 (&r)[4]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int u = threadIdx.x + k * ATT_THREADS, rr = u >> 5, cc = u & 31, p = p0 + rr;
    r[k] = p < c1 ? reinterpret_cast<const uint4*>(base + (size_t)p * HD)[cc] : make_uint4(0, 0, 0, 0);
  }
}

// grid (T, M, NQ / ATT_HB)
template <bool STEP>
__global__ __launch_bounds__(ATT_THREADS) void k_attn_split(AttnPtrs P, AttnGeom gin, const StepDev* sp, int sliding,
                                                            int T) {
  __shared__ AttnGeom g;
  __shared__ float qs[ATT_HB][8][32];              // lane l's 32 query values: s0 chain then s1 chain
  __shared__ __align__(16) uint16_t kt[ATT_TILE][8][40];  // same per-lane order for the keys (80-byte rows)
  __shared__ uint16_t vt[ATT_TILE][HD];
  __shared__ float sw[ATT_HB][ATT_PMAX];
  __shared__ float wmax[ATT_THREADS / 64][ATT_HB];
  __shared__ float smax[ATT_HB], ssum[ATT_HB];
  const int t = blockIdx.x, m = blockIdx.y, h0 = blockIdx.z * ATT_HB;
  if (threadIdx.x == 0) {
    if (STEP) geom_from_step(sp, sliding, T, g);
    else g = gin;
  }
  __syncthreads();
  if (m >= g.M) return;
  // E:740 attn_allowed for this block's row, with the row's bounds held in registers
  const int lo_m = g.lo[m], pos_m = g.pos[m], sl_m = g.skip_lo[m], sh_m = g.skip_hi[m];
  auto allowed = [=](int p) { return p >= lo_m && p <= pos_m && !(p >= sl_m && p <= sh_m); };
  const int len = g.kmax - g.kmin + 1;
  const int c0 = g.kmin + (int)((long)t * len / T), c1 = g.kmin + (int)((long)(t + 1) * len / T);
  const int PP = c1 - c0;
  for (int idx = threadIdx.x; idx < ATT_HB * HD; idx += ATT_THREADS) {
    const int hh = idx / HD, e = idx % HD;  // element e: chain s = (e/8)%2, step tt = e/16, lane e%8
    qs[hh][e & 7][((e >> 3) & 1) * 16 + (e >> 4)] = P.q[(size_t)m * P.ldq + (h0 + hh) * HD + e];
  }
  const int ps = threadIdx.x >> 3, l = threadIdx.x & 7;
  float mymax[ATT_HB];
#pragma unroll
  for (int hh = 0; hh < ATT_HB; ++hh) mymax[hh] = -1e30f;
  __syncthreads();
  float qr[ATT_HB][32];  // this lane's query values of the block's heads
#pragma unroll
  for (int hh = 0; hh < ATT_HB; ++hh)
#pragma unroll
    for (int i = 0; i < 32; ++i) qr[hh][i] = qs[hh][l][i];

  // sweep 1: scores (E:750-816)
  uint4 rk[4];
  if (c0 < c1) tile_fetch(P.KC, c0, c1, rk);
  for (int pb = c0; pb < c1; pb += ATT_TILE) {
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; ++k) {  // scatter the chunk's 8 keys into their lanes' arrays
      const int u = threadIdx.x + k * ATT_THREADS, rr = u >> 5, cc = u & 31;
      const uint32_t w4[4] = {rk[k].x, rk[k].y, rk[k].z, rk[k].w};
      const int slot = (cc & 1) * 16 + (cc >> 1);
#pragma unroll
      for (int e = 0; e < 8; ++e) kt[rr][e][slot] = (uint16_t)(w4[e >> 1] >> (16 * (e & 1)));
    }
    __syncthreads();
    if (pb + ATT_TILE < c1) tile_fetch(P.KC, pb + ATT_TILE, c1, rk);  // next tile in flight
    const int p = pb + ps;
    if (p < c1 && allowed(p)) {
      float kf[32];
      const uint4* kv4 = reinterpret_cast<const uint4*>(&kt[ps][l][0]);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint4 u = kv4[c];
        const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          kf[c * 8 + 2 * e] = as_f32(w4[e] << 16);
          kf[c * 8 + 2 * e + 1] = as_f32(w4[e] & 0xFFFF0000u);
        }
      }
#pragma unroll
      for (int hh = 0; hh < ATT_HB; ++hh) {
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int tt = 0; tt < 16; ++tt) {
          s0 = fmaf(qr[hh][tt], kf[tt], s0);
          s1 = fmaf(qr[hh][16 + tt], kf[16 + tt], s1);
        }
        float v = s0 + s1;
        v = v + __shfl_xor(v, 4, 8);
        v = v + __shfl_xor(v, 1, 8);
        v = v + __shfl_xor(v, 2, 8);
        if (l == 0) {
          sw[hh][p - c0] = v;
          mymax[hh] = (mymax[hh] < v) ? v : mymax[hh];
        }
      }
    }
  }
#pragma unroll
  for (int hh = 0; hh < ATT_HB; ++hh) {
    float v = mymax[hh];
    for (int s = 8; s < 64; s <<= 1) v = fmaxf(v, __shfl_xor(v, s, 64));
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6][hh] = v;
  }
  __syncthreads();
  if (threadIdx.x < ATT_HB) {
    float v = -1e30f;
    for (int w = 0; w < ATT_THREADS / 64; ++w) v = (v < wmax[w][threadIdx.x]) ? wmax[w][threadIdx.x] : v;
    smax[threadIdx.x] = v;
  }
  __syncthreads();
  // weights exp8(score - max) (E:820)
  for (int idx = threadIdx.x; idx < ATT_HB * PP; idx += ATT_THREADS) {
    const int hh = idx / PP, pp = idx % PP;
    if (allowed(c0 + pp)) sw[hh][pp] = exp8(sw[hh][pp] - smax[hh]);
  }
  __syncthreads();
  if (threadIdx.x < ATT_HB) {  // l = sum of the weights in position order (E:821)
    const int hh = threadIdx.x;
    float lsum = 0.f;
    for (int pp = 0; pp < PP; ++pp)
      if (allowed(c0 + pp)) lsum = lsum + sw[hh][pp];
    ssum[hh] = (g.lo[m] > g.pos[m]) ? 0.0f : lsum;
  }
  // sweep 2: o_i = fma chain over positions (E:826-875), V staged tile by tile
  const int i = threadIdx.x;
  float o[ATT_HB];
#pragma unroll
  for (int hh = 0; hh < ATT_HB; ++hh) o[hh] = 0.f;
  uint4 rv[4];
  if (c0 < c1) tile_fetch(P.VC, c0, c1, rv);
  for (int pb = c0; pb < c1; pb += ATT_TILE) {
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int u = threadIdx.x + k * ATT_THREADS, rr = u >> 5, cc = u & 31;
      *reinterpret_cast<uint4*>(&vt[rr][cc * 8]) = rv[k];
    }
    __syncthreads();
    if (pb + ATT_TILE < c1) tile_fetch(P.VC, pb + ATT_TILE, c1, rv);
    const int nt = min(ATT_TILE, c1 - pb);
    for (int pp = 0; pp < nt; ++pp) {
      if (!allowed(pb + pp)) continue;
      const float vv = bf2f(vt[pp][i]);
#pragma unroll
      for (int hh = 0; hh < ATT_HB; ++hh) o[hh] = fmaf(sw[hh][pb + pp - c0], vv, o[hh]);
    }
  }
#pragma unroll
  for (int hh = 0; hh < ATT_HB; ++hh) P.po[(((size_t)t * g.M + m) * NQ + h0 + hh) * HD + i] = o[hh];
  __syncthreads();
  if (threadIdx.x < ATT_HB) {
    P.pm[((size_t)t * g.M + m) * NQ + h0 + threadIdx.x] = smax[threadIdx.x];
    P.pl[((size_t)t * g.M + m) * NQ + h0 + threadIdx.x] = ssum[threadIdx.x];
  }
}

// E:1019-1059, one block per (row m, head h); M from the geometry or the step parameters
__device__ __forceinline__ void merge_body(const AttnPtrs& P, int M, int T) {
  const int m = blockIdx.x, h = blockIdx.y, i = threadIdx.x;
  // every split's partials are loaded up front (independent loads), then folded in split order
  float pl[MAXT], pm[MAXT], po[MAXT];
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    const size_t k = ((size_t)t * M + m) * NQ + h;
    pl[t] = t < T ? P.pl[k] : 0.f;
    pm[t] = t < T ? P.pm[k] : 0.f;
    po[t] = t < T ? P.po[k * HD + i] : 0.f;
  }
  float M0 = -1e30f;
#pragma unroll
  for (int t = 0; t < MAXT; ++t)
    if (t < T && pl[t] > 0) M0 = (M0 < pm[t]) ? pm[t] : M0;
  double l = 0;
  float acc = 0.f, sc[MAXT];
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    sc[t] = 0.f;
    if (t < T && pl[t] > 0) {
      sc[t] = libm_expf_neg(pm[t] - M0, c_expf_tab);
      l = fma((double)pl[t], (double)sc[t], l);
    }
  }
  const float inv = (float)(1.0 / l);
#pragma unroll
  for (int t = 0; t < MAXT; ++t)
    if (t < T && pl[t] > 0) acc = fmaf(po[t], sc[t], acc);
  P.out[(size_t)m * P.ldo + h * HD + i] = r16(acc * inv);
}

__global__ __launch_bounds__(HD) void k_attn_merge(AttnPtrs P, int M, int T) { merge_body(P, M, T); }

__global__ __launch_bounds__(HD) void k_attn_merge_step(AttnPtrs P, const StepDev* sp, int T) {
  if ((int)blockIdx.x >= sp->M) return;
  merge_body(P, sp->M, T);
}

void launch_attn(const uint16_t* KC, const uint16_t* VC, const float* q, const StepDev* sp, int sliding, int T,
                 int ctxcap, float* po, float* pm, float* pl, float* att, int M, hipStream_t st) {
  (void)ctxcap;
  AttnPtrs P{KC, VC, q, NQ * HD, po, pm, pl, att, NQ * HD};
  AttnGeom g{};
  hipLaunchKernelGGL(k_attn_split<true>, dim3(T, M, NQ / ATT_HB), dim3(ATT_THREADS), 0, st, P, g, sp, sliding, T);
  hipLaunchKernelGGL(k_attn_merge_step, dim3(M, NQ), dim3(HD), 0, st, P, sp, T);
}

void launch_attn_geom(const uint16_t* KC, const uint16_t* VC, const float* q, int ldq, const AttnGeom& g,
                      float* po, float* pm, float* pl, float* out, int ldo, hipStream_t st) {
  AttnPtrs P{KC, VC, q, ldq, po, pm, pl, out, ldo};
  hipLaunchKernelGGL(k_attn_split<false>, dim3(g.T, g.M, NQ / ATT_HB), dim3(ATT_THREADS), 0, st, P, g,
                     (const StepDev*)nullptr, 0, g.T);
  hipLaunchKernelGGL(k_attn_merge, dim3(g.M, NQ), dim3(HD), 0, st, P, g.M, g.T);
}

int attn_pmax() { return ATT_PMAX; }

}  // namespace g4v
