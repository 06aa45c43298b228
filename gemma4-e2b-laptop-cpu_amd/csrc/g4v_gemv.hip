// g4v_gemv.hip -- exact-order W4G32 GEMV / skinny GEMM for gfx950.
//
// Reproduces w4::gemm_rows_tile (engine/w4g32_avx2.h:64-96) bit for bit.  For output (m, n)
// the reference keeps 8 fp32 lane accumulators; lane j of group g consumes bytes j and 8+j
// of the group's 16 bytes:
//   a = lo(b_j) * xe[j]; a = fma(lo(b_8+j), xe[8+j], a); a = fma(hi(b_j), xo[j], a);
//   a = fma(hi(b_8+j), xo[8+j], a); row_j = fma(a, sc_g, row_j);  off = fma(sc_g, gsum_g, off)
//   y = ((r0+r4)+(r1+r5))+((r2+r6)+(r3+r7)) - 8 off
// Here each of those 8 accumulators lives in its own GPU lane ("chain lane" (n, j)), so the
// fp32 rounding sequence is the reference's; the 8-lane sum uses xor-shuffles in the same
// tree.  Weights are re-laid once at upload so a lane's two bytes of 8 consecutive groups
// are one coalesced 16-byte load; activations are staged in LDS in the per-lane order
// (xe_j, xe_8+j, xo_j, xo_8+j) with their per-group sums.
//
// Parallelism: a row needs 8 lanes per activation-row slot.  For small N the M activation
// rows are spread over MS lane groups (MS = 1, 2, 4 or 8), multiplying the lanes per
// output row; the decode is repeated per group, the FMA chains are not.
#include "g4v_internal.h"

namespace g4v {

__global__ void k_relayout_w4(const uint8_t* __restrict__ w, uint4* __restrict__ wr, int N, int K) {
  const int GC = K / 256;
  const size_t total = (size_t)N * GC * 8;
  for (size_t u = (size_t)blockIdx.x * blockDim.x + threadIdx.x; u < total;
       u += (size_t)gridDim.x * blockDim.x) {
    const int j = (int)(u & 7);
    const size_t nc = u >> 3;
    const int c = (int)(nc % GC);
    const size_t n = nc / GC;
    const uint8_t* row = w + n * (size_t)(K / 2);
    uint32_t d[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int g0 = 8 * c + 2 * k, g1 = g0 + 1;
      d[k] = (uint32_t)row[g0 * 16 + j] | ((uint32_t)row[g0 * 16 + 8 + j] << 8) |
             ((uint32_t)row[g1 * 16 + j] << 16) | ((uint32_t)row[g1 * 16 + 8 + j] << 24);
    }
    wr[u] = make_uint4(d[0], d[1], d[2], d[3]);
  }
}

void launch_relayout_w4(const uint8_t* w, uint4* wr, int N, int K, hipStream_t st) {
  const size_t total = (size_t)N * (K / 256) * 8;
  int grid = (int)((total + 255) / 256);
  if (grid > 65536) grid = 65536;
  hipLaunchKernelGGL(k_relayout_w4, dim3(grid), dim3(256), 0, st, w, wr, N, K);
}

constexpr int GEMV_THREADS = 256;

// MT: activation rows (template bound), MS: lane groups sharing one output row,
// EPI: epilogue.  Lane index = (rowslot * MS + mslot) * 8 + j.
template <int MT, int MS, int EPI>
__global__ __launch_bounds__(GEMV_THREADS) void k_gemv(GemvArgs a) {
  constexpr int MPL = (MT + MS - 1) / MS;  // activation rows per lane
  constexpr int LPR = 8 * MS;               // lanes per output row
  constexpr int RPW = 64 / LPR;             // output rows per wave
  constexpr int RPB = RPW * (GEMV_THREADS / 64);
  if (a.active && *a.active == 0) return;
  extern __shared__ float4 lds4[];
  const int K = a.K, G = K / 32, GC = K / 256;
  const int M = a.active ? min(a.M, *a.active) : a.M;  // rows beyond a device-side count are idle
  float4* XL = lds4;                               // [MT][G][8]
  float* GS = reinterpret_cast<float*>(lds4 + MT * G * 8);  // [MT][G]
  for (int idx = threadIdx.x; idx < MT * G * 8; idx += GEMV_THREADS) {
    const int j = idx & 7, g = (idx >> 3) % G, m = idx / (G * 8);
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (m < M) {
      const float* b = a.x + (size_t)m * a.ldx + g * 32;
      v = make_float4(b[2 * j], b[16 + 2 * j], b[2 * j + 1], b[17 + 2 * j]);
    }
    XL[idx] = v;
  }
  for (int idx = threadIdx.x; idx < MT * G; idx += GEMV_THREADS) {
    const int g = idx % G, m = idx / G;
    float s = 0.f;
    if (m < M) {
      const float* b = a.x + (size_t)m * a.ldx + g * 32;
      for (int i = 0; i < 32; ++i) s += b[i];  // W:22 sequential group sum
    }
    GS[idx] = s;
  }
  __syncthreads();

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 7, mslot = (lane >> 3) % MS, rslot = lane / LPR;
  const int m0 = mslot * MPL;
  const int moff = m0 + (j < MPL ? j : MPL - 1);  // activation row of this lane's offset chain
  const int ntiles = a.tiles[3];

  for (int t = blockIdx.x; t < ntiles; t += gridDim.x) {
    // which matrix / row this lane serves
    int mi, n;
    if (EPI == EPI_GATEUP) {
      // row slots alternate gate / up for the same n: slot 2p -> gate, 2p+1 -> up
      mi = rslot & 1;
      n = t * (RPB / 2) + wave * (RPW / 2) + (rslot >> 1);
    } else {
      mi = (t >= a.tiles[1]) + (t >= a.tiles[2]);
      n = (t - a.tiles[mi]) * RPB + wave * RPW + rslot;
    }
    const W4Dev W = mi == 0 ? a.mat[0] : (mi == 1 ? a.mat[1] : a.mat[2]);
    const bool valid = n < W.N;
    const uint4* wp = W.wr + ((size_t)(valid ? n : 0) * GC) * 8 + j;
    const uint4* sp = reinterpret_cast<const uint4*>(W.s + (size_t)(valid ? n : 0) * G);

    float row[MPL];
#pragma unroll
    for (int q = 0; q < MPL; ++q) row[q] = 0.f;
    float off = 0.f;

    for (int c = 0; c < GC; ++c) {
      const uint4 wv = valid ? wp[(size_t)c * 8] : make_uint4(0, 0, 0, 0);
      const uint4 sv = valid ? sp[c] : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t d = k == 0 ? wv.x : (k == 1 ? wv.y : (k == 2 ? wv.z : wv.w));
        const uint32_t s2 = k == 0 ? sv.x : (k == 1 ? sv.y : (k == 2 ? sv.z : sv.w));
        const uint32_t lo = d & 0x0F0F0F0Fu, hi = (d >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int g = c * 8 + 2 * k + h;
          const float l0 = (float)((lo >> (16 * h)) & 0xFFu);
          const float l1 = (float)((lo >> (16 * h + 8)) & 0xFFu);
          const float h0 = (float)((hi >> (16 * h)) & 0xFFu);
          const float h1 = (float)((hi >> (16 * h + 8)) & 0xFFu);
          const float sc = h ? as_f32(s2 & 0xFFFF0000u) : as_f32(s2 << 16);
#pragma unroll
          for (int q = 0; q < MPL; ++q) {
            const float4 xv = XL[((m0 + q) * G + g) * 8 + j];
            float av = l0 * xv.x;
            av = fmaf(l1, xv.y, av);
            av = fmaf(h0, xv.z, av);
            av = fmaf(h1, xv.w, av);
            row[q] = fmaf(av, sc, row[q]);
          }
          off = fmaf(sc, GS[moff * G + g], off);
        }
      }
    }
    // 8-lane tree sum per activation row; lane j keeps the sum of row m0 + j
    float mine = 0.f;
#pragma unroll
    for (int q = 0; q < MPL; ++q) {
      float v = row[q];
      v = v + __shfl_xor(v, 4, 8);
      v = v + __shfl_xor(v, 1, 8);
      v = v + __shfl_xor(v, 2, 8);
      if (q == j) mine = v;
    }
    const float y = mine - 8.f * off;
    const int m = m0 + j;
    const bool own = j < MPL && m < M && valid;

    if (EPI == EPI_STORE) {
      if (own) a.y[mi][(size_t)m * a.ldy[mi] + n] = y;
    } else if (EPI == EPI_GATEUP) {
      // E:292-299: act = rbf8(rbf8(gelu8(rbf8 g)) * rbf8 u); the up value is one row slot up
      const float u = __shfl_down(y, LPR, 64);
      if (own && mi == 0) a.y[0][(size_t)m * a.ldy[0] + n] = r16(r16(gelu8(r16(y))) * r16(u));
    } else {  // EPI_SCREEN, E:487-491: L = s - c|h| and U = c|h| + s, both fused
      float L = -INFINITY;
      if (own) {
        const float cf = a.coef[n], hn = a.hn[m];
        L = fmaf(-cf, hn, y);
        a.y[0][(size_t)m * a.ldy[0] + n] = fmaf(cf, hn, y);
      }
      // max over the row slots of this wave that hold the same m (lanes with equal j, mslot)
#pragma unroll
      for (int sft = LPR; sft < 64; sft <<= 1) L = fmaxf(L, __shfl_xor(L, sft, 64));
      if (rslot == 0 && j < MPL && m < M && L > -INFINITY) atomicMax(&a.lmax_key[m], fkey(L));
    }
  }
}

template <int MT, int MS, int EPI>
static void launch_t(const GemvArgs& a, hipStream_t st, int grid_cap) {
  constexpr int MPL = (MT + MS - 1) / MS;
  constexpr int RPW = 64 / (8 * MS);
  constexpr int RPB = RPW * (GEMV_THREADS / 64);
  (void)MPL;
  (void)RPB;
  const int G = a.K / 32;
  const size_t lds = (size_t)MT * G * 8 * sizeof(float4) + (size_t)MT * G * sizeof(float);
  int grid = a.tiles[3];
  if (grid_cap > 0 && grid > grid_cap) grid = grid_cap;
  hipLaunchKernelGGL((k_gemv<MT, MS, EPI>), dim3(grid), dim3(GEMV_THREADS), lds, st, a);
}

template <int MT, int EPI>
static void launch_ms(const GemvArgs& a, int ms, hipStream_t st, int grid_cap) {
  switch (ms) {
    case 1: launch_t<MT, 1, EPI>(a, st, grid_cap); break;
    case 2: if constexpr (MT >= 2) launch_t<MT, 2, EPI>(a, st, grid_cap); break;
    case 4: if constexpr (MT >= 4) launch_t<MT, 4, EPI>(a, st, grid_cap); break;
    default: if constexpr (MT >= 8) launch_t<MT, 8, EPI>(a, st, grid_cap); break;
  }
}

// rows per 256-thread block for a given lane split
static inline int rows_per_block(int ms) { return (64 / (8 * ms)) * (GEMV_THREADS / 64); }

// Pick the lane split: spread activation rows over more lanes while the launch has
// fewer chain lanes than the GPU has SIMD lanes.
static int pick_ms(int MT, int Ntot, int epi) {
  if (epi != EPI_STORE) return 1;
  int ms = 1;
  while (ms < 8 && ms * 2 <= MT && (long)Ntot * 8 * ms < 256L * 64 * 4) ms *= 2;
  return ms;
}

void launch_gemv(const GemvArgs& a_in, int epi, hipStream_t st, int grid_cap) {
  GemvArgs a = a_in;
  const int MT = a.M;
  int Ntot = 0;
  for (int i = 0; i < 3; ++i) Ntot += a.mat[i].N;
  const int ms = pick_ms(MT, Ntot, epi);
  const int rpb = rows_per_block(ms);
  a.tiles[0] = 0;
  if (epi == EPI_GATEUP) {
    a.tiles[1] = a.tiles[2] = a.tiles[3] = (a.mat[0].N + rpb / 2 - 1) / (rpb / 2);
  } else {
    for (int i = 0; i < 3; ++i) a.tiles[i + 1] = a.tiles[i] + (a.mat[i].N + rpb - 1) / rpb;
  }
#define G4V_CASE(mt)                                                  \
  case mt:                                                            \
    if (epi == EPI_STORE) launch_ms<mt, EPI_STORE>(a, ms, st, grid_cap);       \
    else if (epi == EPI_GATEUP) launch_ms<mt, EPI_GATEUP>(a, ms, st, grid_cap); \
    else launch_ms<mt, EPI_SCREEN>(a, ms, st, grid_cap);                        \
    break;
  switch (MT) {
    G4V_CASE(1) G4V_CASE(2) G4V_CASE(3) G4V_CASE(4) G4V_CASE(5) G4V_CASE(6) G4V_CASE(7) G4V_CASE(8)
    default: break;
  }
#undef G4V_CASE
}

}  // namespace g4v
