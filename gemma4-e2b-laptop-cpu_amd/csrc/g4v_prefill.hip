// g4v_prefill.hip -- the prompt pass (prefill) on gfx950: row kernels and the prefill attention.
//
// Restates run_req's prefill loop (E:1594-1599) with ENGINE_PREFILL_INT8=1 for the synthetic
// stack: fwd (E:1256-1405) over blocks of pfb rows.  The rows of every block go through the
// layer in one pass here (layer l of a row needs the KV rows of layer l of the earlier rows
// only, so blocks may share passes); a block's size still picks its attention path:
//   attn_tile (E:1063-1083) when M >= 4 and p0 + M > 64, run_mh (E:1338-1349) otherwise
// (the split-KV case of a short tail block runs through the split kernels of the verify pass).
// The linear layers are the W4A8 matrix-core GEMM (g4v_w4a8.hip); the row kernels below hold the
// norms, RoPE, cache writes and residuals in plain [row][K] layouts.
//
// Prefill attention, per row r at position P (lo = P - 511 clamped at 0 on sliding layers, else
// 0) and query head h, with K, V in the device cache layout (kc_index / vc_index):
//   scores (k_pf_scores): s_p = q . k_p in the path's chain order (attn_tile: two 8-lane FMA
//     chains over hd in steps of 16, summed lane-wise, then hsum; run_mh: one 8-lane chain in
//     steps of 8, then hsum), written to a scratch row [8][P - lo + 1];
//   output (k_pf_attn_out): mx = max_p s_p; attn_tile: w = exp8(s - mx), den = sum w in order,
//     O = fma(w, v, O) in position order, out = r16(O * (1 / den)); run_mh: e = expf(s - mx),
//     den = sum e in order, O = fma(e / den, v, O) in order, out = r16(O).
#include <algorithm>

#include "g4v_layer.h"

namespace g4v {

namespace {

// attention path of row r (E:1305, 1328, 1337): its block [b pfb, ...) of M rows at p0
__device__ __forceinline__ bool pf_tiled(int r, const PfGeom& g) {
  const int b = r / g.pfb, M = min(g.pfb, g.n - b * g.pfb), p0 = g.pos0 + b * g.pfb;
  return g.sib < 0 && M >= 4 && p0 + M > 64;
}
__device__ __forceinline__ int pf_lo(int P, int sliding) { return sliding ? max(0, P - 511) : 0; }
// first key of row r (slot P): the window runs from its RoPE position (pos0 + 1 for the sibling)
__device__ __forceinline__ int pf_row_lo(int r, int P, const PfGeom& g, int sliding) {
  return pf_lo(r == g.sib ? g.pos0 + 1 : P, sliding);
}
// E:1345 valid(p) of row r at slot P
__device__ __forceinline__ bool pf_valid(int r, int P, int p, const PfGeom& g) {
  return r != g.sib || p <= g.pos0 || p == P;
}
// offset of the score row of segment row rr (rows r0 + j, positions Pb + j, Pb = pos0 + r0)
__device__ __forceinline__ long long pf_soff(int rr, int Pb, int sliding) {
  const long long R = rr;
  if (!sliding) return 8 * (R * (Pb + 1) + R * (R - 1) / 2);
  const long long c = min(max(512 - Pb, 0), rr);  // rows whose range starts at 0
  return 8 * (c * (Pb + 1) + c * (c - 1) / 2 + (R - c) * 512);
}

// score row of segment row rr of a launch over nrows rows (the sibling row's, whose window may be
// longer, after all of them)
__device__ __forceinline__ long long pf_srow(int rr, int r, int nrows, int Pb, int sliding, const PfGeom& g) {
  return r == g.sib ? pf_soff(nrows, Pb, sliding) : pf_soff(rr, Pb, sliding);
}

// E:1262-1267: x = r16(E[tok] * sqrt(H)); a = (x * r) * in_ln (unrounded: the W4A8 source)
__global__ __launch_bounds__(ROW_THREADS) void k_pf_embed(const uint16_t* __restrict__ E, const int* __restrict__ toks,
                                                          const float* __restrict__ in_ln, float sqh,
                                                          float* __restrict__ x, float* __restrict__ a) {
  __shared__ __align__(16) float xs[H];
  __shared__ double red[16];
  const int m = blockIdx.x;
  const int tok = toks[m];
  for (int i = threadIdx.x; i < H; i += ROW_THREADS) {
    const float v = r16(bf2f(E[(size_t)tok * H + i]) * sqh);
    xs[i] = v;
    x[(size_t)m * H + i] = v;
  }
  __syncthreads();
  const float r = rms_inv(block_sumsq(xs, H, red), H);
  for (int i = threadIdx.x; i < H; i += ROW_THREADS) a[(size_t)m * H + i] = (xs[i] * r) * in_ln[i];
}

// E:1291-1303 / 1307-1324 for one row: the 8 query heads and k normed with their weights, v
// without, all rounded to bf16 values; NeoX RoPE on q and k at position P; k, v to the cache
// (own = 0: a layer that reads another layer's cache, E:1288, 1304: q only).  D: the head dim.
template <int D>
__global__ __launch_bounds__(D) void k_pf_qkv(float* __restrict__ q, const float* __restrict__ k,
                                              const float* __restrict__ v, const float* __restrict__ qn,
                                              const float* __restrict__ kn, const float* __restrict__ cs,
                                              const float* __restrict__ sn, uint16_t* __restrict__ KC,
                                              uint16_t* __restrict__ VC, int P0, int sib, int own,
                                              const int* __restrict__ dpos) {
  constexpr int NV = NQ + 2;
  if (dpos) P0 = *dpos;  // a captured verify pass: the position from the step parameters
  __shared__ float xv[NV][D];
  __shared__ double part[NV][16];
  __shared__ float rinv[NV];
  const int m = blockIdx.x, e = threadIdx.x, P = P0 + m;
#pragma unroll
  for (int h = 0; h < NQ; ++h) xv[h][e] = q[(size_t)m * NQ * D + h * D + e];
  xv[NQ][e] = own ? k[(size_t)m * D + e] : 0.f;
  xv[NQ + 1][e] = own ? v[(size_t)m * D + e] : 0.f;
  __syncthreads();
  if (e < NV * 16) {  // ss_avx2 order (E:326-343): lane t16 sums x[16 s + t16]^2 over s
    const int row = e >> 4, t16 = e & 15;
    double s = 0;
#pragma unroll
    for (int i = 0; i < D / 16; ++i) {
      const double d = (double)xv[row][16 * i + t16];
      s = fma(d, d, s);
    }
    part[row][t16] = s;
  }
  __syncthreads();
  if (e < NV) {
    const double* p = part[e];
    double a[4];
#pragma unroll
    for (int l = 0; l < 4; ++l) a[l] = (p[l] + p[4 + l]) + (p[8 + l] + p[12 + l]);
    rinv[e] = rms_inv((a[0] + a[2]) + (a[1] + a[3]), D);
  }
  __syncthreads();
  float y[NV];
#pragma unroll
  for (int h = 0; h < NQ; ++h) y[h] = r16((xv[h][e] * rinv[h]) * qn[e]);
  y[NQ] = own ? r16((xv[NQ][e] * rinv[NQ]) * kn[e]) : 0.f;
  y[NQ + 1] = r16(xv[NQ + 1][e] * rinv[NQ + 1]);
  __syncthreads();
#pragma unroll
  for (int h = 0; h < NQ + 1; ++h) xv[h][e] = y[h];
  __syncthreads();
  // E:394-402 NeoX halves: out_i = fma(u, c, -(w s)) and out_{i+D/2} = fma(w, c, u s)
  const int i2 = e & (D / 2 - 1), PR = m == sib ? P0 + 1 : P;  // E:1292 the sibling's RoPE position
  const float c = cs[(size_t)PR * (D / 2) + i2], sv = sn[(size_t)PR * (D / 2) + i2];
  auto rot = [&](const float* yy) {
    return e < D / 2 ? fmaf(yy[e], c, -(yy[e + D / 2] * sv)) : fmaf(yy[e], c, yy[e - D / 2] * sv);
  };
#pragma unroll
  for (int h = 0; h < NQ; ++h) q[(size_t)m * NQ * D + h * D + e] = rot(xv[h]);
  if (own) {
    KC[kc_index_d<D>(P, e)] = f2bf(rot(xv[NQ]));
    VC[vc_index_d<D>(P, e)] = f2bf(y[NQ + 1]);
  }
}

// scores of one row against a span of 256 positions: lane = position, all 8 heads per lane (the
// key row is read and widened once for the 8 heads); the query heads sit in LDS in slot order
// (kc_slot), so every lane of a wave reads the same LDS word (broadcast)
constexpr int PF_SPAN = 256;
template <int D>
__global__ __launch_bounds__(256) void k_pf_scores(const float* __restrict__ q, const uint16_t* __restrict__ KC,
                                                   float* __restrict__ S, PfGeom g, int r0, int sliding,
                                                   const int* __restrict__ dpos) {
  __shared__ __align__(16) float qs[NQ][D];
  if (dpos) g.pos0 = *dpos;  // a captured verify pass: the position from the step parameters
  // the last rows (longest ranges) first, so that the long blocks do not trail the grid
  const int rr = gridDim.x - 1 - blockIdx.x, r = r0 + rr, P = g.pos0 + r, lo = pf_row_lo(r, P, g, sliding);
  const int len = P - lo + 1;
  const int sp0 = lo + blockIdx.y * PF_SPAN;
  if (sp0 > P) return;  // uniform
  const bool tiled = pf_tiled(r, g);
  for (int idx = threadIdx.x; idx < NQ * D; idx += 256) {
    const int h = idx / D, e = idx % D;
    qs[h][kc_slot_d<D>(e)] = q[(size_t)r * NQ * D + idx];
  }
  __syncthreads();
  const int p = sp0 + threadIdx.x;
  if (p > P) return;  // no barrier follows
  const uint16_t* kr = KC + (size_t)p * D;
  constexpr int CL = D / 16;  // steps of one chain
  // sb(l, s, c8): the slot of step 8 c8 of chain (l, s), element 128 c8 + 8 s + l, the first of
  // 8 contiguous slots holding steps 8 c8 .. 8 c8 + 7 (kc_slot_d, either head dim)
  auto sb = [](int l, int s, int c8) { return kc_slot_d<D>(128 * c8 + 8 * s + l); };
  float vv[NQ][8];
  if (tiled) {
    // chain (l, s) = sum over tt of q[16 tt + 8 s + l] k[...], tt in order; vv[h][l] = chain
    // (l, 0) + chain (l, 1)
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      float ch[NQ][2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        float kf[CL];
#pragma unroll
        for (int c8 = 0; c8 < CL / 8; ++c8) {
          const uint4 kk = *reinterpret_cast<const uint4*>(kr + sb(l, s, c8));
          const uint32_t kw[4] = {kk.x, kk.y, kk.z, kk.w};
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            kf[8 * c8 + 2 * c] = as_f32(kw[c] << 16);
            kf[8 * c8 + 2 * c + 1] = as_f32(kw[c] & 0xFFFF0000u);
          }
        }
#pragma unroll
        for (int h = 0; h < NQ; ++h) {
          float a = 0.f;
#pragma unroll
          for (int c8 = 0; c8 < CL / 8; ++c8) {
            const float4* q4 = reinterpret_cast<const float4*>(&qs[h][sb(l, s, c8)]);
#pragma unroll
            for (int c = 0; c < 2; ++c) {
              const float4 qq = q4[c];
              a = fmaf(qq.x, kf[8 * c8 + 4 * c], a);
              a = fmaf(qq.y, kf[8 * c8 + 4 * c + 1], a);
              a = fmaf(qq.z, kf[8 * c8 + 4 * c + 2], a);
              a = fmaf(qq.w, kf[8 * c8 + 4 * c + 3], a);
            }
          }
          ch[h][s] = a;
        }
      }
#pragma unroll
      for (int h = 0; h < NQ; ++h) vv[h][l] = ch[h][0] + ch[h][1];
    }
  } else {
    // chain l over t = 0 .. D/8 - 1 of element 8 t + l = 16 (t >> 1) + 8 (t & 1) + l: chain
    // (l, t & 1)'s step t >> 1; kf[s CL + tt] holds step tt of chain (l, s)
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      float kf[D / 8];
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int c8 = 0; c8 < CL / 8; ++c8) {
          const uint4 kk = *reinterpret_cast<const uint4*>(kr + sb(l, s, c8));
          const uint32_t kw[4] = {kk.x, kk.y, kk.z, kk.w};
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            kf[s * CL + 8 * c8 + 2 * c] = as_f32(kw[c] << 16);
            kf[s * CL + 8 * c8 + 2 * c + 1] = as_f32(kw[c] & 0xFFFF0000u);
          }
        }
#pragma unroll
      for (int h = 0; h < NQ; ++h) {
        float a = 0.f;
#pragma unroll
        for (int t = 0; t < D / 8; ++t) {
          const int s = t & 1, tt = t >> 1;
          a = fmaf(qs[h][sb(l, s, tt >> 3) + (tt & 7)], kf[s * CL + tt], a);
        }
        vv[h][l] = a;
      }
    }
  }
  float* Srow = S + pf_srow(rr, r, gridDim.x, g.pos0 + r0, sliding, g);
  const bool ok = pf_valid(r, P, p, g);  // a skipped position never wins the maximum
#pragma unroll
  for (int h = 0; h < NQ; ++h) Srow[(size_t)h * len + (p - lo)] = ok ? hsum8(vv[h]) : -INFINITY;
}

// output of one row: one wave, lane l holds dims 4l .. 4l+3 of the 8 heads (32 accumulators), so
// each weight read from LDS (wave-uniform) feeds 4 FMAs.  Weights of PF_CP positions at a time
// go to LDS; the value rows are read 8 positions (16 bytes of a dim) at a time where positions
// are 8-aligned, one at a time at the edges of the range
constexpr int PF_CP = 256;  // positions per weight chunk (4 per lane)
template <int D>
__global__ __launch_bounds__(64) void k_pf_attn_out(const float* __restrict__ S, const uint16_t* __restrict__ VC,
                                                    float* __restrict__ att, PfGeom g, int r0, int sliding,
                                                    ExpfTab tab, int staged, const int* __restrict__ dpos) {
  __shared__ __align__(16) float w[NQ][PF_CP];
  if (dpos) g.pos0 = *dpos;
  __shared__ uint64_t T[32];
  // the last rows (longest ranges) first, so that the long blocks do not trail the grid
  const int rr = gridDim.x - 1 - blockIdx.x, r = r0 + rr, P = g.pos0 + r, lo = pf_row_lo(r, P, g, sliding);
  const int len = P - lo + 1;
  const int lane = threadIdx.x;
  const bool tiled = pf_tiled(r, g);
  const float* Srow = S + pf_srow(rr, r, gridDim.x, g.pos0 + r0, sliding, g);
  if (lane < 32) T[lane] = tab.t[lane];
  float mx[NQ];  // max per head (order-free), on every lane
#pragma unroll
  for (int h = 0; h < NQ; ++h) {
    float m = -1e30f;
    for (int jj = lane; jj < len; jj += 64) m = fmaxf(m, Srow[(size_t)h * len + jj]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    mx[h] = m;
  }
  __syncthreads();  // T
  float den = 0.f;  // lanes 0..7: head `lane`'s sum in position order
  if (!tiled) {     // run_mh divides by the sum before the V pass
    for (int c0 = 0; c0 < len; c0 += PF_CP) {
      const int cn = min(PF_CP, len - c0);
#pragma unroll
      for (int k = 0; k < PF_CP / 64; ++k) {
        const int jj = lane + 64 * k;
        if (jj < cn) {
          const bool ok = pf_valid(r, P, lo + c0 + jj, g);  // skipped positions weigh 0 (den + 0 is exact)
#pragma unroll
          for (int h = 0; h < NQ; ++h) w[h][jj] = ok ? libm_expf_neg(Srow[(size_t)h * len + c0 + jj] - mx[h], T) : 0.f;
        }
      }
      __syncthreads();
      if (lane < NQ)
        for (int jj = 0; jj < cn; ++jj) den = den + w[lane][jj];
      __syncthreads();
    }
  }
  float dh[NQ];  // run_mh: the sums, on every lane
#pragma unroll
  for (int h = 0; h < NQ; ++h) dh[h] = __shfl(den, h);
  constexpr int DL = D / 64;  // dims per lane
  float O[NQ][DL];
#pragma unroll
  for (int h = 0; h < NQ; ++h)
#pragma unroll
    for (int d = 0; d < DL; ++d) O[h][d] = 0.f;
  // dim DL lane + d of position p in the cache layout (vc_index_d)
  auto vat = [&](int p, int d) { return VC + vc_index_d<D>(p, DL * lane + d); };
  float sreg[PF_CP / 64][NQ];  // scores of this lane's positions of the next chunk
#pragma unroll
  for (int k = 0; k < PF_CP / 64; ++k)
#pragma unroll
    for (int h = 0; h < NQ; ++h) sreg[k][h] = lane + 64 * k < len ? Srow[(size_t)h * len + lane + 64 * k] : 0.f;
  for (int c0 = 0; c0 < len; c0 += PF_CP) {
    const int cn = min(PF_CP, len - c0);
#pragma unroll
    for (int k = 0; k < PF_CP / 64; ++k) {
      const int jj = lane + 64 * k;
      if (jj < cn) {
        const bool ok = pf_valid(r, P, lo + c0 + jj, g);  // fma(0, v, O) leaves O as it is
#pragma unroll
        for (int h = 0; h < NQ; ++h) {
          const float dd = sreg[k][h] - mx[h];
          w[h][jj] = !ok ? 0.f : (tiled ? exp8(dd) : libm_expf_neg(dd, T) / dh[h]);
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < PF_CP / 64; ++k) {
      const int jj = c0 + PF_CP + lane + 64 * k;
      if (jj < len)
#pragma unroll
        for (int h = 0; h < NQ; ++h) sreg[k][h] = Srow[(size_t)h * len + jj];
    }
    const int pa = lo + c0, pe = pa + cn;  // positions [pa, pe) of this chunk
    const int a8 = min((pa + 7) & ~7, pe), e8 = max(pe & ~7, a8);
    for (int p = pa; p < a8; ++p) {        // leading positions up to an 8-boundary
      float v[DL];
#pragma unroll
      for (int d = 0; d < DL; ++d) v[d] = bf2f(*vat(p, d));
#pragma unroll
      for (int h = 0; h < NQ; ++h) {
        const float ww = w[h][p - pa];
#pragma unroll
        for (int d = 0; d < DL; ++d) O[h][d] = fmaf(ww, v[d], O[h][d]);
      }
    }
    for (int p = a8; p < e8; p += 8) {     // 8 positions of each of the lane's 4 dims
      uint4 vq[DL];
#pragma unroll
      for (int d = 0; d < DL; ++d) vq[d] = *reinterpret_cast<const uint4*>(vat(p, d));
      const int j0 = p - pa;
#pragma unroll
      for (int t2 = 0; t2 < 4; ++t2) {     // positions j0 + 2 t2, j0 + 2 t2 + 1
        float va[DL], vb[DL];
#pragma unroll
        for (int d = 0; d < DL; ++d) {
          const uint32_t u = t2 == 0 ? vq[d].x : (t2 == 1 ? vq[d].y : (t2 == 2 ? vq[d].z : vq[d].w));
          va[d] = as_f32(u << 16);
          vb[d] = as_f32(u & 0xFFFF0000u);
        }
#pragma unroll
        for (int h = 0; h < NQ; ++h) {
          const float wa = w[h][j0 + 2 * t2], wb = w[h][j0 + 2 * t2 + 1];  // j0 may be odd
#pragma unroll
          for (int d = 0; d < DL; ++d) O[h][d] = fmaf(wa, va[d], O[h][d]);
#pragma unroll
          for (int d = 0; d < DL; ++d) O[h][d] = fmaf(wb, vb[d], O[h][d]);
        }
      }
    }
    for (int p = e8; p < pe; ++p) {        // trailing positions
      float v[DL];
#pragma unroll
      for (int d = 0; d < DL; ++d) v[d] = bf2f(*vat(p, d));
#pragma unroll
      for (int h = 0; h < NQ; ++h) {
        const float ww = w[h][p - pa];
#pragma unroll
        for (int d = 0; d < DL; ++d) O[h][d] = fmaf(ww, v[d], O[h][d]);
      }
    }
    if (tiled && lane < NQ)
      for (int jj = 0; jj < cn; ++jj) den = den + w[lane][jj];
    __syncthreads();
  }
  const float inv = tiled ? 1.0f / den : 1.0f;  // lanes 0..7
  float* orow = att + (size_t)r * NQ * D;
#pragma unroll
  for (int h = 0; h < NQ; ++h) {
    const float ih = __shfl(inv, h);
    float v[DL];
#pragma unroll
    for (int d = 0; d < DL; ++d) v[d] = tiled ? r16(O[h][d] * ih) : r16(O[h][d]);
    const int n0 = h * D + DL * lane;
    if (staged) {  // the staged GEMV input layout of the o projection (staged_index)
#pragma unroll
      for (int d = 0; d < DL; ++d) orow[staged_index(n0 + d)] = v[d];
    } else {
#pragma unroll
      for (int d4 = 0; d4 < DL; d4 += 4)
        *reinterpret_cast<float4*>(orow + n0 + d4) = make_float4(v[d4], v[d4 + 1], v[d4 + 2], v[d4 + 3]);
    }
  }
}

// The same output for a pass of few rows (a verify pass, M <= 8): one block per (row, head), one
// output dim per thread, so that every dim's chain over the positions has a thread of its own
// (the kernel above gives a whole row to one wave).  Arithmetic as above: the max over the row's
// scores; run_mh: den = the sum in position order of libm expf(s - max) (one thread, chunk by
// chunk), w = expf(s - max) / den, out = r16(fma chain of w v in position order); attn_tile:
// w = exp8(s - max), out = r16(chain * (1 / den)) with den the sum of w in order.  Weights are
// staged per chunk of PF_RC positions from the 8-aligned position at or below lo, 0 where not
// valid, so the value reads take 8 positions (16 bytes of a dim) at a time; a zero weight leaves
// the chain unchanged (its value is taken as +0 and the chain is never -0).
constexpr int PF_RC = 512;
template <int D>
__global__ __launch_bounds__(D) void k_pf_attn_rows(const float* __restrict__ S, const uint16_t* __restrict__ VC,
                                                   float* __restrict__ att, PfGeom g, int r0, int sliding,
                                                   ExpfTab tab, int staged, const int* __restrict__ dpos) {
  __shared__ __align__(16) float w[PF_RC];
  if (dpos) g.pos0 = *dpos;
  __shared__ uint64_t T[32];
  __shared__ float red[D / 64];
  __shared__ float dens;
  const int rr = gridDim.x - 1 - blockIdx.x, r = r0 + rr, P = g.pos0 + r, lo = pf_row_lo(r, P, g, sliding);
  const int h = blockIdx.y, d = threadIdx.x;
  const int len = P - lo + 1;
  const bool tiled = pf_tiled(r, g);
  const float* Sh = S + pf_srow(rr, r, gridDim.x, g.pos0 + r0, sliding, g) + (size_t)h * len;
  if (d < 32) T[d] = tab.t[d];
  float mx = -1e30f;  // order free
  for (int jj = d; jj < len; jj += D) mx = fmaxf(mx, Sh[jj]);
  for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if ((d & 63) == 0) red[d >> 6] = mx;
  __syncthreads();
  mx = red[0];
#pragma unroll
  for (int k = 1; k < D / 64; ++k) mx = fmaxf(mx, red[k]);
  const int pa = lo & ~7, pend = P + 1;  // chunks cover [pa, P]; slots before lo weigh 0
  float den = 0.f;                        // thread 0: the sum in position order
  if (!tiled) {  // run_mh divides by the sum before the value pass
    for (int c0 = pa; c0 < pend; c0 += PF_RC) {
      const int cn = min(PF_RC, pend - c0);
      __syncthreads();  // the previous chunk's weights are summed
      for (int j = d; j < cn; j += D) {
        const int p = c0 + j;
        w[j] = (p >= lo && pf_valid(r, P, p, g)) ? libm_expf_neg(Sh[p - lo] - mx, T) : 0.f;
      }
      __syncthreads();
      if (d == 0)
        for (int j = 0; j < cn; ++j) den = den + w[j];
    }
    if (d == 0) dens = den;
    __syncthreads();
    den = dens;
  }
  // the cache parts of 32 positions up to the one holding P (within the slab of kv_cap positions)
  const __amdgpu_buffer_rsrc_t vrs = buf_rsrc(VC, (uint32_t)((P >> 5) + 1) * (32 * D * 2));
  float O = 0.f;
  for (int c0 = pa; c0 < pend; c0 += PF_RC) {
    constexpr int VR = 8;  // value steps in flight
    const int cn = min(PF_RC, pend - c0);
    const int n8 = (cn + 7) >> 3, nv = (n8 + VR - 1) / VR * VR;  // steps of 8 positions; 8 nv <= PF_RC
    __syncthreads();  // the previous chunk is used
    for (int j = d; j < 8 * nv; j += D) {
      const int p = c0 + j;
      float v = 0.f;
      if (j < cn && p >= lo && pf_valid(r, P, p, g)) {
        const float dd = Sh[p - lo] - mx;
        v = tiled ? exp8(dd) : libm_expf_neg(dd, T) / den;
      }
      w[j] = v;
    }
    __syncthreads();
    // the value words of 8 positions of dim d (16 contiguous bytes of the cache), VR steps in
    // flight with no branch between a load and its use; the steps past n8 read positions past P
    // (zeros beyond P's 32-position part, stale words within it) and weigh 0.  attn_tile's den =
    // the sum of the weights in position order runs in every lane beside the value chain (the
    // zero weights leave it unchanged)
    auto load_v = [&](int j) {
      const int p8 = c0 + 8 * j;
      return buf_load16(vrs, (uint32_t)((p8 >> 5) * (32 * D) + ((p8 >> 3) & 3) * (8 * D)) * 2 + d * 16);
    };
    uint4 ring[VR];
#pragma unroll
    for (int i = 0; i < VR; ++i) {  // in slot order, as the loop reloads them
      ring[i] = load_v(i);
      __builtin_amdgcn_sched_barrier(0);
    }
    for (int jb = 0; jb < nv; jb += VR) {
#pragma unroll
      for (int i = 0; i < VR; ++i) {
        // the slot's words are unpacked before its next load is issued into the same registers
        // (a value live across that load would make the ring rotate through copies)
        const uint32_t u4[4] = {ring[i].x, ring[i].y, ring[i].z, ring[i].w};
        float v8[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) v8[k] = as_f32((k & 1) ? (u4[k >> 1] & 0xFFFF0000u) : (u4[k >> 1] << 16));
        __builtin_amdgcn_sched_barrier(0);
        ring[i] = load_v(jb + VR + i);
        __builtin_amdgcn_sched_barrier(0);  // issued here, VR steps ahead of its use
        const int j8 = 8 * (jb + i);
        const float4 wa = *reinterpret_cast<const float4*>(&w[j8]);
        const float4 wb = *reinterpret_cast<const float4*>(&w[j8 + 4]);
        const float w8[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float vv = w8[k] != 0.f ? v8[k] : 0.f;
          O = fmaf(w8[k], vv, O);
          if (tiled) den = den + w8[k];
        }
      }
    }
  }
  const float y = tiled ? r16(O * (1.0f / den)) : r16(O);
  float* orow = att + (size_t)r * NQ * D;
  const int n = h * D + d;
  orow[staged ? staged_index(n) : n] = y;
}

// E:1358-1361 (W4A8 source kept): o = r16(o); tmp = rms(o, post_attn); x = r16(x + r16(tmp));
// a = r16(rms(x, pre_ff))
__global__ __launch_bounds__(ROW_THREADS) void k_pf_post_attn(const float* __restrict__ o, float* __restrict__ x,
                                                              float* __restrict__ a, const float* __restrict__ w1,
                                                              const float* __restrict__ w2) {
  __shared__ __align__(16) float os[H];
  __shared__ __align__(16) float xs[H];
  __shared__ double red[16];
  const int m = blockIdx.x;
  for (int i = threadIdx.x; i < H; i += ROW_THREADS) os[i] = r16(o[(size_t)m * H + i]);
  __syncthreads();
  const float r1 = rms_inv(block_sumsq(os, H, red), H);
  for (int i = threadIdx.x; i < H; i += ROW_THREADS) {
    const float v = r16(x[(size_t)m * H + i] + r16((os[i] * r1) * w1[i]));
    xs[i] = v;
    x[(size_t)m * H + i] = v;
  }
  __syncthreads();
  const float r2 = rms_inv(block_sumsq(xs, H, red), H);
  for (int i = threadIdx.x; i < H; i += ROW_THREADS) a[(size_t)m * H + i] = r16((xs[i] * r2) * w2[i]);
}

// E:1369-1370: act = r16(r16(gelu8(r16 g)) * r16 u)
__global__ void k_pf_act(const float* __restrict__ g, const float* __restrict__ u, float* __restrict__ act, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    act[i] = r16(r16(gelu8(r16(g[i]))) * r16(u[i]));
}

// E:1375-1404 with a zero per-layer-embedding branch: o = r16(o); tmp = rms(o, post_ff);
// x = r16(x + r16(tmp)); x = r16(x * scalar); then a = rms(x, next in_ln) (unrounded) or, after
// the last layer and for rows m >= hrow (hrow >= 0), h[m - hrow] = r16(rms(x, fnorm)) and, when
// hn is given, hn[m - hrow] = |h| (E:1417).  The same block with the per-layer-input branch
// (E:1387-1404) takes the per_layer_projection output as o and post_per_layer_input_norm as w1;
// with scalar 1, no next norm and hrow -1 it is the plain residual block of E:1375-1377.
__global__ __launch_bounds__(ROW_THREADS) void k_pf_post_ff(const float* __restrict__ o, float* __restrict__ x,
                                                            float* __restrict__ a, const float* __restrict__ w1,
                                                            const float* __restrict__ next_in_ln,
                                                            const float* __restrict__ fnorm, float scalar,
                                                            float* __restrict__ h, int hrow, float* __restrict__ hn) {
  __shared__ __align__(16) float os[H];
  __shared__ __align__(16) float xs[H];
  __shared__ double red[16];
  const int m = blockIdx.x;
  for (int i = threadIdx.x; i < H; i += ROW_THREADS) os[i] = r16(o[(size_t)m * H + i]);
  __syncthreads();
  const float r1 = rms_inv(block_sumsq(os, H, red), H);
  for (int i = threadIdx.x; i < H; i += ROW_THREADS) {
    float v = r16(x[(size_t)m * H + i] + r16((os[i] * r1) * w1[i]));
    v = r16(v * scalar);
    xs[i] = v;
    x[(size_t)m * H + i] = v;
  }
  if (!next_in_ln && (hrow < 0 || m < hrow)) return;  // uniform
  __syncthreads();
  const float r2 = rms_inv(block_sumsq(xs, H, red), H);
  if (next_in_ln) {
    for (int i = threadIdx.x; i < H; i += ROW_THREADS) a[(size_t)m * H + i] = (xs[i] * r2) * next_in_ln[i];
  } else {
    float* hr = h + (size_t)(m - hrow) * H;
    for (int i = threadIdx.x; i < H; i += ROW_THREADS) {
      const float v = r16((xs[i] * r2) * fnorm[i]);
      os[i] = v;
      hr[i] = v;
    }
    if (!hn) return;  // uniform
    __syncthreads();
    const double ss = block_sumsq(os, H, red);
    if (threadIdx.x == 0) hn[m - hrow] = (float)sqrt(ss);
  }
}

// E:615-660 ple_fused_task after its product, one block per (row m, layer l): pr = the
// per_layer_model_projection row (8960 = 35 x 256), prl = r16(pr_l / sqrt(1536)),
// pj = rms(prl, per_layer_projection_norm), pli_l = (pj + r16(16 PLE[tok][l])) * 0.70710678118
__global__ __launch_bounds__(256) void k_gm_ple(const float* __restrict__ pr, const int* __restrict__ toks,
                                                const uint16_t* __restrict__ ple, const float* __restrict__ plnorm,
                                                float* __restrict__ pli) {
  constexpr int PD = 256, NLG = 35;
  __shared__ float xs[PD];
  __shared__ double red[16];
  const int m = blockIdx.x, l = blockIdx.y, i = threadIdx.x;
  const size_t base = (size_t)m * NLG * PD + (size_t)l * PD;
  const float s1 = 1.0f / sqrtf((float)H);
  xs[i] = r16(pr[base + i] * s1);
  __syncthreads();
  const float r = rms_inv(block_sumsq(xs, PD, red), PD);
  const float pj = (xs[i] * r) * plnorm[i];
  const float pev = r16(bf2f(ple[(size_t)toks[m] * NLG * PD + (size_t)l * PD + i]) * 16.0f);
  pli[base + i] = (pj + pev) * 0.70710678118f;
}

// E:405-443 pg_fused_task after its product: g2 = r16(r16(gelu8(r16 pgv)) * r16(pli_l)), rows of 256
__global__ void k_gm_pg_act(const float* __restrict__ pgv, const float* __restrict__ pli, int l, int M,
                            float* __restrict__ g2) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= M * 256) return;
  const int m = idx >> 8, i = idx & 255;
  g2[idx] = r16(r16(gelu8(r16(pgv[idx]))) * r16(pli[(size_t)m * 35 * 256 + (size_t)l * 256 + i]));
}

}  // namespace

void launch_pf_embed(const uint16_t* E, const int* toks, const float* in_ln, float sqh, float* x, float* a, int M,
                     hipStream_t st) {
  hipLaunchKernelGGL(k_pf_embed, dim3(M), dim3(ROW_THREADS), 0, st, E, toks, in_ln, sqh, x, a);
}
void launch_pf_qkv(float* q, const float* k, const float* v, const float* qn, const float* kn, const float* cs,
                   const float* sn, uint16_t* KC, uint16_t* VC, int P0, int M, hipStream_t st, int sib, int hd,
                   int own, const int* dpos) {
  if (hd == 512)
    hipLaunchKernelGGL(k_pf_qkv<512>, dim3(M), dim3(512), 0, st, q, k, v, qn, kn, cs, sn, KC, VC, P0, sib, own, dpos);
  else
    hipLaunchKernelGGL(k_pf_qkv<HD>, dim3(M), dim3(HD), 0, st, q, k, v, qn, kn, cs, sn, KC, VC, P0, sib, own, dpos);
}
long long pf_score_floats(int M, int Pb, int sliding) {
  const long long R = M;
  if (!sliding) return 8 * (R * (Pb + 1) + R * (R - 1) / 2);
  const long long c = std::min<long long>(std::max(512 - Pb, 0), R);
  return 8 * (c * (Pb + 1) + c * (c - 1) / 2 + (R - c) * 512);
}
void launch_pf_attn(const float* q, const uint16_t* KC, const uint16_t* VC, float* S, float* att, const PfGeom& g,
                    int r0, int M, int sliding, hipStream_t st, bool staged, int hd, const int* dpos, int maxpos) {
  // (dpos: the position comes from device memory; the grid then covers positions below maxpos,
  // and the score blocks past a row's range return at once)
  const int Plast = dpos ? maxpos - 1 : g.pos0 + r0 + M - 1;
  // the sibling's window (from pos0 + 1) can be longer than 512 by the rows it skips
  const int maxlen = sliding ? std::min(Plast + 1, g.sib >= 0 ? r0 + M - 1 + 511 : 512) : Plast + 1;
  const int spans = (maxlen + PF_SPAN - 1) / PF_SPAN;
  ExpfTab tab{G4V_EXPF_TABLE};
  // a pass of few rows gives every (row, head) a block; a prompt block keeps a wave per row (it
  // reads each value row once for the 8 heads)
  const bool rows = M <= MAXM;
  if (hd == 512) {
    hipLaunchKernelGGL(k_pf_scores<512>, dim3(M, spans), dim3(256), 0, st, q, KC, S, g, r0, sliding, dpos);
    if (rows)
      hipLaunchKernelGGL(k_pf_attn_rows<512>, dim3(M, NQ), dim3(512), 0, st, S, VC, att, g, r0, sliding, tab,
                         staged ? 1 : 0, dpos);
    else
      hipLaunchKernelGGL(k_pf_attn_out<512>, dim3(M), dim3(64), 0, st, S, VC, att, g, r0, sliding, tab, staged ? 1 : 0, dpos);
  } else {
    hipLaunchKernelGGL(k_pf_scores<HD>, dim3(M, spans), dim3(256), 0, st, q, KC, S, g, r0, sliding, dpos);
    if (rows)
      hipLaunchKernelGGL(k_pf_attn_rows<HD>, dim3(M, NQ), dim3(HD), 0, st, S, VC, att, g, r0, sliding, tab,
                         staged ? 1 : 0, dpos);
    else
      hipLaunchKernelGGL(k_pf_attn_out<HD>, dim3(M), dim3(64), 0, st, S, VC, att, g, r0, sliding, tab, staged ? 1 : 0, dpos);
  }
}
void launch_pf_post_attn(const float* o, float* x, float* a, const float* w1, const float* w2, int M, hipStream_t st) {
  hipLaunchKernelGGL(k_pf_post_attn, dim3(M), dim3(ROW_THREADS), 0, st, o, x, a, w1, w2);
}
void launch_pf_act(const float* g, const float* u, float* act, size_t n, hipStream_t st) {
  const int grid = (int)std::min<size_t>((n + 255) / 256, 8192);
  hipLaunchKernelGGL(k_pf_act, dim3(grid), dim3(256), 0, st, g, u, act, n);
}
void launch_pf_post_ff(const float* o, float* x, float* a, const float* w1, const float* next_in_ln,
                       const float* fnorm, float scalar, float* h, int hrow, int M, hipStream_t st, float* hn) {
  hipLaunchKernelGGL(k_pf_post_ff, dim3(M), dim3(ROW_THREADS), 0, st, o, x, a, w1, next_in_ln, fnorm, scalar, h,
                     hrow, hn);
}
void launch_gm_ple(const float* pr, const int* toks, const uint16_t* ple, const float* plnorm, float* pli, int M,
                   hipStream_t st) {
  hipLaunchKernelGGL(k_gm_ple, dim3(M, 35), dim3(256), 0, st, pr, toks, ple, plnorm, pli);
}
void launch_gm_pg_act(const float* pgv, const float* pli, int l, int M, float* g2, hipStream_t st) {
  hipLaunchKernelGGL(k_gm_pg_act, dim3((M * 256 + 255) / 256), dim3(256), 0, st, pgv, pli, l, M, g2);
}

}  // namespace g4v
