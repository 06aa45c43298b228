// g4v_head.hip -- certified head screen, exact rescore and greedy argmax on gfx950.
//
// Reference path (E = engine/gemma4_engine.cpp, X3 = engine/bf16_exp3_head.h):
//   screen  E:460-538   s = W4G32(screen, h); L = s - c|h|, U = c|h| + s (fused)
//   select  E:1453-1466 thr = calc_thr(max L) (E:1410-1414); survivors {U >= thr}; more than
//                       30,000 -> full head (E:1489-1498)
//   rescore E:540-571   exp3 dot in the X3:83-107 lane order, exceptions added after the
//                       8-lane sum, v = r16(y)
//   argmax  E:1467-1468 / E:1496  lowest index with v >= max - 2 and cap(v) == cap(max),
//                       cap(v) = r16(30 tanh(v / 30)) read from a LUT over bf16 inputs.
// The exp3 head is held on the device as the bf16 weights its decoder yields ("dec16",
// lane order j, 16+j, 8+j, 24+j per group) plus the same exception list (CSR by row).
#include <algorithm>

#include "g4v_internal.h"
#include "g4v_head.h"

namespace g4v {

__device__ __forceinline__ float cap_of(float v, const uint16_t* lut) { return bf2f(lut[as_u32(v) >> 16]); }

// E:454-459 / E:1410-1414 calc_thr with the cap LUT (all cap arguments are bf16 values)
__device__ float calc_thr_dev(float L, const uint16_t* lut) {
  const float Lr = r16(L), cmL = cap_of(Lr, lut);
  float lo = Lr - 64.0f, hi = Lr;
  for (int it = 0; it < 40; ++it) {
    const float mid = 0.5f * (lo + hi);
    if (cap_of(r16(mid), lut) == cmL) hi = mid;
    else lo = mid;
  }
  return hi - 0.25f;
}

__global__ void k_head_reset(HeadScratch hs, int MT) {
  const int m = threadIdx.x;
  if (m < MT) {
    hs.cnt[m] = 0;
    hs.lmax_key[m] = fkey(-INFINITY);
    hs.vmax_key[m] = fkey(-INFINITY);
    hs.best[m] = 0x7fffffff;
  }
}

// one block: max L over the screen's per-block partials, then calc_thr with the cap table
// staged in LDS (the 40 bisection steps would otherwise be 40 dependent global loads)
constexpr int THR_THREADS = 1024;
__global__ __launch_bounds__(THR_THREADS) void k_head_thr(HeadScratch hs, const uint16_t* __restrict__ lut, int MT,
                                                          int nb, const int* active) {
  if (active && *active == 0) return;
  const int MA = active ? min(MT, *active) : MT;
  extern __shared__ uint4 lds_lut4[];
  uint16_t* L16 = reinterpret_cast<uint16_t*>(lds_lut4);
  __shared__ float red[THR_THREADS / 64][MAXM];
  const uint4* g4 = reinterpret_cast<const uint4*>(lut);
  for (int i = threadIdx.x; i < 65536 / 8; i += THR_THREADS) lds_lut4[i] = g4[i];
  for (int m = 0; m < MA; ++m) {
    float v = -INFINITY;
    for (int i = threadIdx.x; i < nb; i += THR_THREADS) v = fmaxf(v, hs.lpart[(size_t)m * nb + i]);
    for (int s = 1; s < 64; s <<= 1) v = fmaxf(v, __shfl_xor(v, s, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6][m] = v;
  }
  __syncthreads();
  if (threadIdx.x < MA) {
    float v = -INFINITY;
    for (int w = 0; w < THR_THREADS / 64; ++w) v = fmaxf(v, red[w][threadIdx.x]);
    hs.thr[threadIdx.x] = calc_thr_dev(v, L16);
  }
}

// survivors {U >= calc_thr(max L)}, unordered; counts beyond the limit are kept for the decision
__global__ void k_head_select(HeadScratch hs, int MT, int V, const int* active) {
  if (active && *active == 0) return;
  // rows at or beyond a device-side count stay at zero survivors (and so never fall back)
  const int MA = active ? min(MT, *active) : MT;
  __shared__ float thr[MAXM];
  if (threadIdx.x < MA) thr[threadIdx.x] = hs.thr[threadIdx.x];
  __syncthreads();
  // One counter update per block and row: the block counts its survivors, reserves that many
  // slots with one atomic, and writes them there (the list order is free: the rescore and the
  // tie rule do not depend on it).  The block covers a contiguous range of rows.
  __shared__ int wtot[8], base_s;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int per = (V + gridDim.x - 1) / gridDim.x;
  const int n0 = blockIdx.x * per, n1 = min(V, n0 + per);
  for (int m = 0; m < MA; ++m) {
    const float* U = hs.u + (size_t)m * V;
    const float tm = thr[m];
    int c = 0;
    for (int n = n0 + threadIdx.x; n < n1; n += blockDim.x) c += U[n] >= tm;
    int inc = c;  // inclusive scan within the wave
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(inc, o);
      if (lane >= o) inc += v;
    }
    if (lane == 63) wtot[wv] = inc;
    __syncthreads();
    int before = 0, total = 0;
    for (int w = 0; w < nw; ++w) {
      before += w < wv ? wtot[w] : 0;
      total += wtot[w];
    }
    if (threadIdx.x == 0) base_s = total ? atomicAdd(&hs.cnt[m], total) : 0;
    __syncthreads();
    int p = base_s + before + inc - c;
    if (c)
      for (int n = n0 + threadIdx.x; n < n1; n += blockDim.x)
        if (U[n] >= tm) {
          if (p < HEAD_LIMIT) hs.list[(size_t)m * HEAD_LIMIT + p] = n;
          ++p;
        }
    __syncthreads();  // wtot / base_s are reused by the next row
  }
}

// Exact dot of dec16 row n with x (LDS float4 per (g, j) = x[32g+j], x[32g+16+j], x[32g+8+j],
// x[32g+24+j]); lanes j = 0..7 of the calling group hold the 8 accumulators.  Returns the
// tree-summed value in every lane of the group.
__device__ __forceinline__ float dec_dot(const uint4* __restrict__ dec, size_t n, int j,
                                         const float4* xh) {
  float acc = 0.f;
  const uint4* p = dec + n * (size_t)(24 * 8) + j;
#pragma unroll 4
  for (int q = 0; q < 24; ++q) {
    const uint4 w = p[q * 8];
    const float4 x0 = xh[(2 * q) * 8 + j], x1 = xh[(2 * q + 1) * 8 + j];
    acc = fmaf(as_f32(w.x << 16), x0.x, acc);
    acc = fmaf(as_f32(w.x & 0xFFFF0000u), x0.y, acc);
    acc = fmaf(as_f32(w.y << 16), x0.z, acc);
    acc = fmaf(as_f32(w.y & 0xFFFF0000u), x0.w, acc);
    acc = fmaf(as_f32(w.z << 16), x1.x, acc);
    acc = fmaf(as_f32(w.z & 0xFFFF0000u), x1.y, acc);
    acc = fmaf(as_f32(w.w << 16), x1.z, acc);
    acc = fmaf(as_f32(w.w & 0xFFFF0000u), x1.w, acc);
  }
  float v = acc;
  v = v + __shfl_xor(v, 4, 8);
  v = v + __shfl_xor(v, 1, 8);
  v = v + __shfl_xor(v, 2, 8);
  return v;
}

// stage h rows in the dec16 lane order plus the raw rows (for the exception chain)
__device__ __forceinline__ void stage_h(const float* __restrict__ h, int MT, float4* XH, float* XR) {
  for (int idx = threadIdx.x; idx < MT * 48 * 8; idx += blockDim.x) {
    const int j = idx & 7, g = (idx >> 3) % 48, m = idx / (48 * 8);
    const float* b = h + (size_t)m * H + g * 32;
    XH[idx] = make_float4(b[j], b[16 + j], b[8 + j], b[24 + j]);
  }
  for (int idx = threadIdx.x; idx < MT * H; idx += blockDim.x) XR[idx] = h[idx];
  __syncthreads();
}

// rescore the survivors of rows whose count is within the limit; 8 lanes per survivor
__global__ __launch_bounds__(256) void k_head_rescore(HeadScratch hs, HeadDev hd, const float* __restrict__ h,
                                                      int MT, const int* active) {
  if (active && *active == 0) return;
  extern __shared__ float4 lds4[];
  float4* XH = lds4;
  float* XR = reinterpret_cast<float*>(lds4 + MT * 48 * 8);
  int tot = 0, cnt[MAXM];
  for (int m = 0; m < MT; ++m) {
    const int c = hs.cnt[m];
    cnt[m] = c <= HEAD_LIMIT ? c : 0;
    tot += cnt[m];
  }
  if (tot == 0) return;
  stage_h(h, MT, XH, XR);
  const int j = threadIdx.x & 7, slot = threadIdx.x >> 3, nslots = blockDim.x >> 3;
  for (int it = blockIdx.x * nslots + slot; it < tot + (nslots - 1); it += gridDim.x * nslots) {
    // (m, idx) of item `it`; items past the end compute row 0 and store nothing
    int m = 0, idx = it;
    while (m < MT - 1 && idx >= cnt[m]) idx -= cnt[m++];
    const bool ok = it < tot && idx < cnt[m];
    const int n = ok ? hs.list[(size_t)m * HEAD_LIMIT + idx] : 0;
    float y = dec_dot(hd.dec, (size_t)n, j, XH + m * 48 * 8);
    if (ok && j == 0) {
      for (int e = hd.exc_ptr[n]; e < hd.exc_ptr[n + 1]; ++e) y = fmaf(hd.exc_del[e], XR[m * H + hd.exc_col[e]], y);
      const float v = r16(y);
      hs.sval[(size_t)m * HEAD_LIMIT + idx] = v;
      atomicMax(&hs.vmax_key[m], fkey(v));
    }
  }
}

// full head for the rows whose survivor count exceeds the limit (E:1489-1498); the dec16 row
// is read once for all MT activation rows.  This pass stores each row's main dot (X3:83-107,
// before the exception deltas); k_head_exc then adds the deltas in order and rounds.
// the 8 weights of one (row, group pair, lane) entry of the exp3 form (HeadDev::x3sm / x3ix):
// exponent bytes from the 8-entry codebook by byte permutes, then the bf16 bit patterns
// (hi = sign | e >> 1, lo = (e & 1) << 7 | mantissa) moved to the top of each fp32 word
__device__ __forceinline__ void x3_decode(uint2 sm, uint32_t ix, uint32_t cblo, uint32_t cbhi, float (&w)[8]) {
  const uint32_t ee = __builtin_amdgcn_perm(cbhi, cblo, ix & 0x0F0F0F0Fu);
  const uint32_t eo = __builtin_amdgcn_perm(cbhi, cblo, (ix >> 4) & 0x0F0F0F0Fu);
  const uint32_t he = (sm.x & 0x80808080u) | ((ee >> 1) & 0x7F7F7F7Fu), le = ((ee << 7) & 0x80808080u) | (sm.x & 0x7F7F7F7Fu);
  const uint32_t ho = (sm.y & 0x80808080u) | ((eo >> 1) & 0x7F7F7F7Fu), lo = ((eo << 7) & 0x80808080u) | (sm.y & 0x7F7F7F7Fu);
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const uint32_t sel = ((uint32_t)(4 + b) << 24) | ((uint32_t)b << 16) | 0x0C0Cu;
    w[2 * b] = as_f32(__builtin_amdgcn_perm(he, le, sel));
    w[2 * b + 1] = as_f32(__builtin_amdgcn_perm(ho, lo, sel));
  }
}

// the exp3 form from the decoded head (every decoded exponent is a codebook entry)
__global__ void k_x3_pack(HeadDev hd, int V) {
  uint8_t cb[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) cb[i] = hd.cb[i];
  const size_t total = (size_t)V * 24 * 8;
  for (size_t u = (size_t)blockIdx.x * blockDim.x + threadIdx.x; u < total; u += (size_t)gridDim.x * blockDim.x) {
    const uint4 v = hd.dec[u];
    const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
    uint32_t se = 0, so = 0, ix = 0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t b = (wd[k >> 1] >> (16 * (k & 1))) & 0xFFFFu;
      const uint32_t smb = ((b >> 8) & 0x80u) | (b & 0x7Fu), e = (b >> 7) & 0xFFu;
      uint32_t idx = 0;
#pragma unroll
      for (int i = 7; i >= 0; --i)
        if (cb[i] == e) idx = i;
      const int sh = 8 * (k >> 1);
      if (k & 1) {
        so |= smb << sh;
        ix |= idx << (sh + 4);
      } else {
        se |= smb << sh;
        ix |= idx << sh;
      }
    }
    hd.x3smw[u] = make_uint2(se, so);
    hd.x3ixw[u] = ix;
  }
}

template <int MT>
__global__ __launch_bounds__(256) void k_head_full(HeadScratch hs, HeadDev hd, const float* __restrict__ h,
                                                   int V, const int* active) {
  if (active && *active == 0) return;
  extern __shared__ float4 lds4[];
  float4* XH = lds4;
  float* XR = reinterpret_cast<float*>(lds4 + MT * 48 * 8);
  bool any = false;
  bool fb[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    fb[m] = hs.cnt[m] > HEAD_LIMIT;
    any |= fb[m];
  }
  if (!any) return;
  stage_h(h, MT, XH, XR);
  const uint32_t cblo = reinterpret_cast<const uint32_t*>(hd.cb)[0], cbhi = reinterpret_cast<const uint32_t*>(hd.cb)[1];
  const int j = threadIdx.x & 7, slot = threadIdx.x >> 3, nslots = blockDim.x >> 3;
  for (int n0 = blockIdx.x * nslots; n0 < V; n0 += gridDim.x * nslots) {
    const int n = n0 + slot;
    const bool ok = n < V;
    const int nn = ok ? n : 0;
    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0.f;
    const uint2* ps = hd.x3sm + (size_t)nn * (24 * 8) + j;
    const uint32_t* pi = hd.x3ix + (size_t)nn * (24 * 8) + j;
#pragma unroll 8
    for (int q = 0; q < 24; ++q) {
      float wd[8];
      x3_decode(ps[q * 8], pi[q * 8], cblo, cbhi, wd);
      const float w0 = wd[0], w1 = wd[1], w2 = wd[2], w3 = wd[3], w4 = wd[4], w5 = wd[5], w6 = wd[6], w7 = wd[7];
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const float4 x0 = XH[(m * 48 + 2 * q) * 8 + j], x1 = XH[(m * 48 + 2 * q + 1) * 8 + j];
        float a = acc[m];
        a = fmaf(w0, x0.x, a);
        a = fmaf(w1, x0.y, a);
        a = fmaf(w2, x0.z, a);
        a = fmaf(w3, x0.w, a);
        a = fmaf(w4, x1.x, a);
        a = fmaf(w5, x1.y, a);
        a = fmaf(w6, x1.z, a);
        a = fmaf(w7, x1.w, a);
        acc[m] = a;
      }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if (!fb[m]) continue;
      float y = acc[m];
      y = y + __shfl_xor(y, 4, 8);
      y = y + __shfl_xor(y, 1, 8);
      y = y + __shfl_xor(y, 2, 8);
      if (j == 0 && ok) hs.u[(size_t)m * V + n] = y;
    }
  }
}

// X3:103 / E:565 the exception deltas of each row after its main dot, in list order, then the
// bf16 rounding of the logit (E:1494); one thread per row.  One partial max per block and row
// (reduced by the tie kernel).
template <int MT>
__global__ __launch_bounds__(256) void k_head_exc(HeadScratch hs, HeadDev hd, const float* __restrict__ h, int V,
                                                  const int* active) {
  if (active && *active == 0) return;
  extern __shared__ float4 lds4[];
  float4* XH = lds4;
  float* XR = reinterpret_cast<float*>(lds4 + MT * 48 * 8);
  bool any = false;
  bool fb[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    fb[m] = hs.cnt[m] > HEAD_LIMIT;
    any |= fb[m];
  }
  if (!any) return;
  stage_h(h, MT, XH, XR);
  float vrun[MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) vrun[m] = -INFINITY;
  for (int n = blockIdx.x * blockDim.x + threadIdx.x; n < V; n += gridDim.x * blockDim.x) {
    const int e0 = hd.exc_ptr[n], e1 = hd.exc_ptr[n + 1];
    float y[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) y[m] = fb[m] ? hs.u[(size_t)m * V + n] : 0.f;
    for (int e = e0; e < e1; e += 4) {  // four entries per round trip, applied in order
      float dl[4];
      int cl[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int ek = min(e + k, e1 - 1);
        dl[k] = hd.exc_del[ek];
        cl[k] = hd.exc_col[ek];
      }
#pragma unroll
      for (int k = 0; k < 4; ++k)
        if (e + k < e1) {
#pragma unroll
          for (int m = 0; m < MT; ++m) y[m] = fmaf(dl[k], XR[m * H + cl[k]], y[m]);
        }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m)
      if (fb[m]) {
        const float v = r16(y[m]);
        hs.u[(size_t)m * V + n] = v;
        vrun[m] = fmaxf(vrun[m], v);
      }
  }
  __shared__ float red[256 / 64][MT];
#pragma unroll
  for (int m = 0; m < MT; ++m) {
    float v = vrun[m];
    for (int s = 1; s < 64; s <<= 1) v = fmaxf(v, __shfl_xor(v, s, 64));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6][m] = v;
  }
  __syncthreads();
  if (threadIdx.x < MT) {
    float v = -INFINITY;
    for (int w = 0; w < 256 / 64; ++w) v = fmaxf(v, red[w][threadIdx.x]);
    hs.vpart[(size_t)threadIdx.x * gridDim.x + blockIdx.x] = v;
  }
}

// lowest index satisfying the tie rule, over survivors or over the full-head logits
__global__ void k_head_tie(HeadScratch hs, const uint16_t* __restrict__ lut, int MT, int V, int nbf,
                           const int* active) {
  if (active && *active == 0) return;
  __shared__ float red[4];
  for (int m = 0; m < MT; ++m) {
    float mx = fkey_inv(hs.vmax_key[m]);
    if (hs.cnt[m] > HEAD_LIMIT) {  // full head: reduce its per-block maxima
      float v = -INFINITY;
      for (int i = threadIdx.x; i < nbf; i += blockDim.x) v = fmaxf(v, hs.vpart[(size_t)m * nbf + i]);
      for (int s = 1; s < 64; s <<= 1) v = fmaxf(v, __shfl_xor(v, s, 64));
      if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
      __syncthreads();
      mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
      __syncthreads();
    }
    const float cm = cap_of(mx, lut);
    int best = 0x7fffffff;
    if (hs.cnt[m] > HEAD_LIMIT) {
      const float* lg = hs.u + (size_t)m * V;
      for (int n = blockIdx.x * blockDim.x + threadIdx.x; n < V; n += gridDim.x * blockDim.x) {
        const float v = lg[n];
        if (v >= mx - 2.0f && cap_of(v, lut) == cm) {
          best = n;
          break;  // later n in this thread's stride are larger
        }
      }
    } else {
      const int c = hs.cnt[m];
      for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < c; i += gridDim.x * blockDim.x) {
        const float v = hs.sval[(size_t)m * HEAD_LIMIT + i];
        const int n = hs.list[(size_t)m * HEAD_LIMIT + i];
        if (v >= mx - 2.0f && cap_of(v, lut) == cm && n < best) best = n;
      }
    }
    if (best != 0x7fffffff) atomicMin(&hs.best[m], best);
  }
}

// ---------------------------------------------------------------------------------------
// head build (one-time): exponent histogram, dec16 + exception list, certified screen
// ---------------------------------------------------------------------------------------
__global__ void k_exp_hist(const uint16_t* __restrict__ E, size_t n, unsigned long long* hist) {
  __shared__ unsigned int lh[256];
  for (int i = threadIdx.x; i < 256; i += blockDim.x) lh[i] = 0;
  __syncthreads();
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    atomicAdd(&lh[(E[i] >> 7) & 0xFF], 1u);
  __syncthreads();
  for (int i = threadIdx.x; i < 256; i += blockDim.x)
    if (lh[i]) atomicAdd(&hist[i], (unsigned long long)lh[i]);
}

// X3:34-39: exact codebook index, else the first nearest exponent (an exception)
__device__ __forceinline__ int cb_index(const uint8_t* cb, int e, bool& exc) {
  for (int i = 0; i < 8; ++i)
    if (cb[i] == e) {
      exc = false;
      return i;
    }
  int best = 0, bd = 1 << 30;
  for (int i = 0; i < 8; ++i) {
    const int dd = abs((int)cb[i] - e);
    if (dd < bd) {
      bd = dd;
      best = i;
    }
  }
  exc = true;
  return best;
}

__device__ __forceinline__ uint16_t dec_weight(uint16_t w, const uint8_t* cb, bool& exc) {
  const int e = (w >> 7) & 0xFF;
  const int idx = cb_index(cb, e, exc);
  return (uint16_t)((w & 0x8000) | ((uint16_t)cb[idx] << 7) | (w & 0x7F));
}

// one thread per (row, group pair): dec16 words in lane order and the per-group exception count
__global__ void k_dec16(const uint16_t* __restrict__ E, HeadDev hd, uint8_t* __restrict__ gcnt, int V) {
  const size_t total = (size_t)V * 24;
  for (size_t u = (size_t)blockIdx.x * blockDim.x + threadIdx.x; u < total; u += (size_t)gridDim.x * blockDim.x) {
    const size_t n = u / 24;
    const int p = (int)(u % 24);
    uint16_t d[2][32];
    for (int gg = 0; gg < 2; ++gg) {
      const int g = 2 * p + gg;
      int c = 0;
      for (int k = 0; k < 32; ++k) {
        bool exc;
        d[gg][k] = dec_weight(E[n * H + g * 32 + k], hd.cb, exc);
        c += exc;
      }
      gcnt[n * 48 + g] = (uint8_t)c;
    }
    uint4* out = hd.decw + (n * 24 + p) * 8;
    for (int j = 0; j < 8; ++j) {
      uint4 v;
      v.x = (uint32_t)d[0][j] | ((uint32_t)d[0][16 + j] << 16);
      v.y = (uint32_t)d[0][8 + j] | ((uint32_t)d[0][24 + j] << 16);
      v.z = (uint32_t)d[1][j] | ((uint32_t)d[1][16 + j] << 16);
      v.w = (uint32_t)d[1][8 + j] | ((uint32_t)d[1][24 + j] << 16);
      out[j] = v;
    }
  }
}

__global__ void k_rowcount(const uint8_t* __restrict__ gcnt, int* __restrict__ rowcnt, int V) {
  for (int n = blockIdx.x * blockDim.x + threadIdx.x; n < V; n += gridDim.x * blockDim.x) {
    int s = 0;
    for (int g = 0; g < 48; ++g) s += gcnt[(size_t)n * 48 + g];
    rowcnt[n] = s;
  }
}

// exceptions of row n in column order: col and exact delta w - dec (X3:39)
__global__ void k_exc_fill(const uint16_t* __restrict__ E, HeadDev hd, int V) {
  for (int n = blockIdx.x * blockDim.x + threadIdx.x; n < V; n += gridDim.x * blockDim.x) {
    int at = hd.exc_ptr[n];
    for (int k = 0; k < H; ++k) {
      const uint16_t w = E[(size_t)n * H + k];
      bool exc;
      const uint16_t dw = dec_weight(w, hd.cb, exc);
      if (exc) {
        hd.exc_col_w[at] = (uint16_t)k;
        hd.exc_del_w[at] = bf2f(w) - bf2f(dw);
        ++at;
      }
    }
  }
}

// E:1236-1243 certified screen build, one thread per row; Wq in the reference's byte layout
__global__ void k_screen_build(const uint16_t* __restrict__ E, uint8_t* __restrict__ Wq,
                               uint16_t* __restrict__ Sq, float* __restrict__ coef, int V) {
  for (int n = blockIdx.x * blockDim.x + threadIdx.x; n < V; n += gridDim.x * blockDim.x) {
    double e2 = 0, w2 = 0;
    for (int g = 0; g < 48; ++g) {
      float w[32], amax = 0.f;
      for (int i = 0; i < 32; ++i) {
        w[i] = bf2f(E[(size_t)n * H + g * 32 + i]);
        const float a = fabsf(w[i]);
        amax = (amax < a) ? a : amax;
      }
      const uint16_t sb = f2bf(amax / 7.0f);
      const float sc = bf2f(sb);
      Sq[(size_t)n * 48 + g] = sb;
      int qv[32];
      for (int i = 0; i < 32; ++i) {
        int v = sc > 0 ? (int)rintf(w[i] / sc) : 0;
        v = v < -8 ? -8 : (v > 7 ? 7 : v);
        qv[i] = v + 8;
        const double d = fma(-(double)v, (double)sc, (double)w[i]);
        e2 = fma(d, d, e2);
        w2 = fma((double)w[i], (double)w[i], w2);
      }
      for (int i = 0; i < 16; ++i) Wq[(size_t)n * 768 + g * 16 + i] = (uint8_t)(qv[2 * i] | (qv[2 * i + 1] << 4));
    }
    coef[n] = (float)fma(1e-4, sqrt(w2), sqrt(e2));  // GCC contracts the reference's sum
  }
}

// ---------------------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------------------
static inline int grid_for(size_t n, int bs, int cap = 16384) {
  size_t g = (n + bs - 1) / bs;
  return (int)(g > (size_t)cap ? cap : (g < 1 ? 1 : g));
}

void head_build(const uint16_t* E, int V, HeadDev& hd, HeadBuildTmp& tmp, hipStream_t st) {
  hipLaunchKernelGGL(k_exp_hist, dim3(1024), dim3(256), 0, st, E, (size_t)V * H, tmp.hist);
}

void head_build_dec(const uint16_t* E, int V, HeadDev& hd, HeadBuildTmp& tmp, hipStream_t st) {
  hipLaunchKernelGGL(k_dec16, dim3(grid_for((size_t)V * 24, 256)), dim3(256), 0, st, E, hd, tmp.gcnt, V);
  hipLaunchKernelGGL(k_rowcount, dim3(grid_for(V, 256)), dim3(256), 0, st, tmp.gcnt, tmp.rowcnt, V);
}

void head_build_x3(int V, HeadDev& hd, hipStream_t st) {
  hipLaunchKernelGGL(k_x3_pack, dim3(grid_for((size_t)V * 24 * 8, 256)), dim3(256), 0, st, hd, V);
}

void head_build_exc(const uint16_t* E, int V, HeadDev& hd, hipStream_t st) {
  hipLaunchKernelGGL(k_exc_fill, dim3(grid_for(V, 256)), dim3(256), 0, st, E, hd, V);
}

void screen_build(const uint16_t* E, int V, uint8_t* Wq, uint16_t* Sq, float* coef, hipStream_t st) {
  hipLaunchKernelGGL(k_screen_build, dim3(grid_for(V, 256)), dim3(256), 0, st, E, Wq, Sq, coef, V);
}

size_t head_lds(int MT) { return (size_t)MT * 48 * 8 * sizeof(float4) + (size_t)MT * H * sizeof(float); }

void head_run(const HeadRun& r, hipStream_t st) {
  const int MT = r.MT, V = r.V;
  // pass-2 launches (rows chosen on the device) are booked under one tag of their own
  auto mark = [&](int tag, int begin, double bytes) {
    if (r.prof.mark) r.prof.mark(r.prof.ctx, r.pass2 ? PT_HEAD2 : tag, begin, bytes);
  };
  hipLaunchKernelGGL(k_head_reset, dim3(1), dim3(64), 0, st, r.hs, MT);
  GemvArgs a{};
  a.mat[0] = r.screen;
  a.y[0] = r.hs.u;
  a.ldy[0] = V;
  a.x = r.h;
  a.ldx = H;
  a.K = H;
  a.M = MT;
  a.coef = r.coef;
  a.hn = r.hn;
  a.lpart = r.hs.lpart;
  a.active = r.active;
  const int cap = std::min(r.grid_cap > 0 ? r.grid_cap : HEAD_MAXGRID, HEAD_MAXGRID);
  mark(PT_HEAD_SCREEN, 1, 0);
  const int nb = launch_gemv(a, EPI_SCREEN, st, cap);
  mark(PT_HEAD_SCREEN, 0, (double)V * (H / 2 + H / 16 + 4));
  mark(PT_HEAD_SELECT, 1, 0);
  static bool thr_lds = false;
  if (!thr_lds) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_head_thr), hipFuncAttributeMaxDynamicSharedMemorySize,
                              65536 * 2);
    thr_lds = true;
  }
  hipLaunchKernelGGL(k_head_thr, dim3(1), dim3(THR_THREADS), 65536 * 2, st, r.hs, r.lut, MT, nb, r.active);
  hipLaunchKernelGGL(k_head_select, dim3(std::min(256, (V + 255) / 256)), dim3(256), 0, st, r.hs, MT, V, r.active);
  mark(PT_HEAD_SELECT, 0, (double)V * 4 * MT);
  mark(PT_HEAD_RESCORE, 1, 0);
  static bool big_lds = false;  // rows 6 to 8 stage more than 64 KB
  if (!big_lds) {
    const void* fns[] = {reinterpret_cast<const void*>(&k_head_rescore), reinterpret_cast<const void*>(&k_head_full<6>),
                         reinterpret_cast<const void*>(&k_head_full<7>), reinterpret_cast<const void*>(&k_head_full<8>),
                         reinterpret_cast<const void*>(&k_head_exc<6>), reinterpret_cast<const void*>(&k_head_exc<7>),
                         reinterpret_cast<const void*>(&k_head_exc<8>)};
    for (const void* f : fns) (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)head_lds(MAXM));
    big_lds = true;
  }
  hipLaunchKernelGGL(k_head_rescore, dim3(256), dim3(256), head_lds(MT), st, r.hs, r.hd, r.h, MT, r.active);
  mark(PT_HEAD_RESCORE, 0, 0);
  const dim3 gf(grid_for(V, 32, cap)), ge(grid_for(V, 256, cap));
  mark(PT_HEAD_FULL, 1, 0);
#define G4V_HEAD_ROWS(mt)                                                                                       \
  case mt:                                                                                                     \
    hipLaunchKernelGGL(k_head_full<mt>, gf, dim3(256), head_lds(mt), st, r.hs, r.hd, r.h, V, r.active);       \
    hipLaunchKernelGGL(k_head_exc<mt>, ge, dim3(256), head_lds(mt), st, r.hs, r.hd, r.h, V, r.active);        \
    break;
  switch (MT) {
    G4V_HEAD_ROWS(1) G4V_HEAD_ROWS(2) G4V_HEAD_ROWS(3) G4V_HEAD_ROWS(4)
    G4V_HEAD_ROWS(5) G4V_HEAD_ROWS(6) G4V_HEAD_ROWS(7) G4V_HEAD_ROWS(8)
    default: break;
  }
#undef G4V_HEAD_ROWS
  mark(PT_HEAD_FULL, 0, r.full_bytes);
  mark(PT_HEAD_TIE, 1, 0);
  hipLaunchKernelGGL(k_head_tie, dim3(grid_for(V, 256, 1024)), dim3(256), 0, st, r.hs, r.lut, MT, V, (int)ge.x,
                     r.active);
  mark(PT_HEAD_TIE, 0, 0);
}

}  // namespace g4v
