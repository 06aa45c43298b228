// g4v_layer.hip -- RMSNorm row kernels, branch selection and acceptance for one verify pass
// on gfx950 (the q/k norm, RoPE and cache write of E:1307-1324 run inside the attention
// kernel, g4v_attn.hip).
//
// References (E = engine/gemma4_engine.cpp): embedding E:1262-1267; residual/norm blocks
// E:1358-1361, E:1375-1404; lazy head + acceptance E:1453-1488, E:1647-1661.
#include <algorithm>

#include "g4v_layer.h"

namespace g4v {


// Write a K-vector held in LDS (v, 16-byte aligned) as one row of the staged GEMV input
// layout (staged_index) plus its group sums, each the sequential fp32 sum of the group's 32
// values (W:22), so the consuming GEMV stages it with plain 16-byte copies.
__device__ void write_staged(const float* v, int K, float* xs, float* gs) {
  float4* xs4 = reinterpret_cast<float4*>(xs);
  for (int idx = threadIdx.x; idx < K / 4; idx += blockDim.x) {
    const float* b = v + (idx >> 3) * 32;
    const int j = idx & 7;
    xs4[idx] = make_float4(b[2 * j], b[16 + 2 * j], b[2 * j + 1], b[17 + 2 * j]);
  }
  for (int g = threadIdx.x; g < K / 32; g += blockDim.x) {
    const float4* b4 = reinterpret_cast<const float4*>(v + g * 32);
    float4 r[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = b4[i];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) s = (((s + r[i].x) + r[i].y) + r[i].z) + r[i].w;
    gs[g] = s;
  }
}

// E:1262-1267: x = rbf8(E[tok] * sqrt(H)); xa = (x * r) * in_ln, xa written staged (+ sums).
// Also gathers the step's RoPE factors: ropestep[ty][m] = the (cos, sin) rows of the layer-type ty
// tables at the row's position, in the order of the attention's 16-lane rows (lane n: cos then
// sin of elements 16 tt + n, tt < 8), so the attention kernel reads them without a dependent load.
__global__ __launch_bounds__(ROW_THREADS) void k_embed(const uint16_t* __restrict__ E, const StepDev* sp,
                                                       const float* __restrict__ in_ln, float sqh,
                                                       float* __restrict__ x, float* __restrict__ xa,
                                                       float* __restrict__ xgs, const float* __restrict__ rope,
                                                       int ctxcap, float* __restrict__ ropestep) {
  __shared__ __align__(16) float xs[H];
  __shared__ __align__(16) float ys[H];
  __shared__ double red[16];
  const int m = blockIdx.x;
  const int tok = sp->toks[m];
  {
    const int ty = threadIdx.x >> 7, i = threadIdx.x & (HD / 2 - 1), rp = sp->rope[m];
    const float* cs = rope + (size_t)(2 * ty) * ctxcap * (HD / 2);
    const float* sn = cs + (size_t)ctxcap * (HD / 2);
    // lane n = i % 16 of a 16-lane row holds elements 16 tt + n, tt < 8 of the rotation's first
    // half: its 8 cos then 8 sin factors at n * 16
    float* dst = ropestep + ((size_t)ty * MAXM + m) * HD + (i & 15) * 16 + (i >> 4);
    dst[0] = cs[(size_t)rp * (HD / 2) + i];
    dst[8] = sn[(size_t)rp * (HD / 2) + i];
  }
  for (int i = threadIdx.x; i < H; i += ROW_THREADS) {
    const float v = r16(bf2f(E[(size_t)tok * H + i]) * sqh);
    xs[i] = v;
    x[(size_t)m * H + i] = v;
  }
  __syncthreads();
  const float r = rms_inv(block_sumsq(xs, H, red), H);
  for (int i = threadIdx.x; i < H; i += ROW_THREADS) ys[i] = (xs[i] * r) * in_ln[i];
  __syncthreads();
  write_staged(ys, H, xa + (size_t)m * H, xgs + (size_t)m * (H / 32));
}

// E:1358-1361: o = r16(o); tmp = rms(o, post_attn); x = r16(x + r16(tmp)); xa = r16(rms(x, pre_ff)).
// Every global input of the row is loaded up front (one round trip), xa is written staged.
constexpr int RPT = H / ROW_THREADS;  // elements of a row per thread
__global__ __launch_bounds__(ROW_THREADS) void k_post_attn(const float* __restrict__ o, float* __restrict__ x,
                                                           float* __restrict__ xa, float* __restrict__ xgs,
                                                           LayerNorms ln) {
  __shared__ __align__(16) float os[H];
  __shared__ __align__(16) float xs[H];
  __shared__ double red[16];
  const int m = blockIdx.x;
  float ov[RPT], xv[RPT], w1[RPT], w2[RPT];
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    const int i = threadIdx.x + k * ROW_THREADS;
    ov[k] = o[(size_t)m * H + i];
    xv[k] = x[(size_t)m * H + i];
    w1[k] = ln.post_attn[i];
    w2[k] = ln.pre_ff[i];
  }
#pragma unroll
  for (int k = 0; k < RPT; ++k) os[threadIdx.x + k * ROW_THREADS] = r16(ov[k]);
  __syncthreads();
  const float r1 = rms_inv(block_sumsq(os, H, red), H);
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    const int i = threadIdx.x + k * ROW_THREADS;
    const float tmp = (os[i] * r1) * w1[k];
    const float v = r16(xv[k] + r16(tmp));
    xs[i] = v;
    x[(size_t)m * H + i] = v;
  }
  __syncthreads();
  const float r2 = rms_inv(block_sumsq(xs, H, red), H);
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    const int i = threadIdx.x + k * ROW_THREADS;
    os[i] = r16((xs[i] * r2) * w2[k]);
  }
  __syncthreads();
  write_staged(os, H, xa + (size_t)m * H, xgs + (size_t)m * (H / 32));
}

// E:1375-1378 and E:1390-1404 with a zero per-layer-embedding branch:
// o = r16(o); tmp = rms(o, post_ff); x = r16(x + r16(tmp)); x = r16(x * scalar);
// then xa = rms(x, next in_ln) (staged) or, after the last layer, h = r16(rms(x, fnorm)), hn = |h|.
__global__ __launch_bounds__(ROW_THREADS) void k_post_ff(const float* __restrict__ o, float* __restrict__ x,
                                                         float* __restrict__ xa, float* __restrict__ xgs,
                                                         LayerNorms ln, const float* __restrict__ next_in_ln,
                                                         const float* __restrict__ fnorm, float* __restrict__ h,
                                                         float* __restrict__ hn) {
  __shared__ __align__(16) float os[H];
  __shared__ __align__(16) float xs[H];
  __shared__ double red[16];
  const int m = blockIdx.x;
  const float* w2p = next_in_ln ? next_in_ln : fnorm;
  float ov[RPT], xv[RPT], w1[RPT], w2[RPT];
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    const int i = threadIdx.x + k * ROW_THREADS;
    ov[k] = o[(size_t)m * H + i];
    xv[k] = x[(size_t)m * H + i];
    w1[k] = ln.post_ff[i];
    w2[k] = w2p[i];
  }
#pragma unroll
  for (int k = 0; k < RPT; ++k) os[threadIdx.x + k * ROW_THREADS] = r16(ov[k]);
  __syncthreads();
  const float r1 = rms_inv(block_sumsq(os, H, red), H);
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    const int i = threadIdx.x + k * ROW_THREADS;
    const float tmp = (os[i] * r1) * w1[k];
    float v = r16(xv[k] + r16(tmp));
    v = r16(v * ln.scalar);
    xs[i] = v;
    x[(size_t)m * H + i] = v;
  }
  __syncthreads();
  const float r2 = rms_inv(block_sumsq(xs, H, red), H);
  if (next_in_ln) {
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int i = threadIdx.x + k * ROW_THREADS;
      os[i] = (xs[i] * r2) * w2[k];
    }
    __syncthreads();
    write_staged(os, H, xa + (size_t)m * H, xgs + (size_t)m * (H / 32));
  } else {
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int i = threadIdx.x + k * ROW_THREADS;
      const float v = r16((xs[i] * r2) * w2[k]);
      os[i] = v;
      h[(size_t)m * H + i] = v;
    }
    __syncthreads();
    const double ss = block_sumsq(os, H, red);
    if (threadIdx.x == 0) hn[m] = (float)sqrt(ss);  // E:1417
  }
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
    } else if (sp->nb >= 1 && sp->b_ok && sp->toks[sp->na + 1] == G0) {
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
// (cache slabs of kvcap positions in the device layout; element i of each row)
__global__ void k_kv_compact(const StepDev* sp, const VerifyResultDev* res, uint16_t* KC, uint16_t* VC, int kvcap) {
  if (res->branch != 1) return;
  const int l = blockIdx.x, i = threadIdx.x;
  uint16_t* K = KC + (size_t)l * kvcap * HD;
  uint16_t* V = VC + (size_t)l * kvcap * HD;
  for (int r = 1; r < res->ncommit; ++r) {
    const int ps = sp->pos0 + res->hrows[r], pd = sp->pos0 + r;
    K[(size_t)pd * HD + i] = K[(size_t)ps * HD + i];  // a key row is one contiguous permuted row
    V[vc_index(pd, i)] = V[vc_index(ps, i)];
  }
}

template <int D>
__global__ void k_kv_compact_d(const StepDev* sp, const VerifyResultDev* res, uint16_t* K, uint16_t* V) {
  if (res->branch != 1) return;
  const int i = threadIdx.x;
  for (int r = 1; r < res->ncommit; ++r) {
    const int ps = sp->pos0 + res->hrows[r], pd = sp->pos0 + r;
    K[(size_t)pd * D + i] = K[(size_t)ps * D + i];
    V[vc_index_d<D>(pd, i)] = V[vc_index_d<D>(ps, i)];
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

// a 256-vector into the 16-lane head order (head16_index)
__global__ void k_perm16(const float* __restrict__ src, float* __restrict__ dst) {
  dst[head16_index(threadIdx.x)] = src[threadIdx.x];
}
void launch_perm16(const float* src, float* dst, hipStream_t st) {
  hipLaunchKernelGGL(k_perm16, dim3(1), dim3(HD), 0, st, src, dst);
}

// ---------------------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------------------
void launch_embed(const uint16_t* E, const StepDev* sp, const float* in_ln, float sqh, float* x, float* xa, float* xgs,
                  const float* rope, int ctxcap, float* ropestep, int M, hipStream_t st) {
  hipLaunchKernelGGL(k_embed, dim3(M), dim3(ROW_THREADS), 0, st, E, sp, in_ln, sqh, x, xa, xgs, rope, ctxcap,
                     ropestep);
}
void launch_post_attn(const float* o, float* x, float* xa, float* xgs, const LayerNorms& ln, int M, hipStream_t st) {
  hipLaunchKernelGGL(k_post_attn, dim3(M), dim3(ROW_THREADS), 0, st, o, x, xa, xgs, ln);
}
void launch_post_ff(const float* o, float* x, float* xa, float* xgs, const LayerNorms& ln, const float* next_in_ln,
                    const float* fnorm, float* h, float* hn, int M, hipStream_t st) {
  hipLaunchKernelGGL(k_post_ff, dim3(M), dim3(ROW_THREADS), 0, st, o, x, xa, xgs, ln, next_in_ln, fnorm, h, hn);
}
void launch_branch(const StepDev* sp, const int* best1, const float* h, const float* hn, float* h2, float* hn2,
                   VerifyResultDev* res, hipStream_t st) {
  hipLaunchKernelGGL(k_branch, dim3(1), dim3(256), 0, st, sp, best1, h, hn, h2, hn2, res);
}
void launch_accept(const StepDev* sp, const int* best1, const int* best2, const int* cnt1, const int* cnt2,
                   VerifyResultDev* res, uint16_t* KC, uint16_t* VC, int NL, int kvcap, hipStream_t st) {
  hipLaunchKernelGGL(k_accept, dim3(1), dim3(64), 0, st, sp, best1, best2, cnt1, cnt2, res);
  if (NL > 0) hipLaunchKernelGGL(k_kv_compact, dim3(NL), dim3(HD), 0, st, sp, res, KC, VC, kvcap);
}
void launch_kv_compact_hd(const StepDev* sp, const VerifyResultDev* res, uint16_t* K, uint16_t* V, int hd,
                          hipStream_t st) {
  if (hd == 512) hipLaunchKernelGGL(k_kv_compact_d<512>, dim3(1), dim3(512), 0, st, sp, res, K, V);
  else hipLaunchKernelGGL(k_kv_compact_d<HD>, dim3(1), dim3(HD), 0, st, sp, res, K, V);
}
// exchange two KV slabs (uint4 words): the prefix cache's slot switch
__global__ void k_swap16(uint4* __restrict__ a, uint4* __restrict__ b, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const uint4 x = a[i];
    a[i] = b[i];
    b[i] = x;
  }
}
void launch_swap16(void* a, void* b, size_t bytes, hipStream_t st) {
  const size_t n = bytes / 16;
  const int grid = (int)std::min<size_t>((n + 255) / 256, 8192);
  if (n) hipLaunchKernelGGL(k_swap16, dim3(grid), dim3(256), 0, st, (uint4*)a, (uint4*)b, n);
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
