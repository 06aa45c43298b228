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
// ("a chunk") are one coalesced 16-byte load; activations are staged in LDS in the per-lane
// order (xe_j, xe_8+j, xo_j, xo_8+j) with their per-group sums.
//
// Parallelism and latency: a row needs 8 lanes per activation-row slot.  For small N the M
// activation rows are spread over MS lane groups (MS = 1, 2, 4 or 8); the decode is
// repeated per group, the FMA chains are not.  Chunks are fetched in batches of four,
// double-buffered, so eight chunks per lane are in flight.  When the activations of all M
// rows do not fit the LDS budget, K is staged in phases; the chains simply continue across
// phases, so the result does not depend on the phase size.
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
constexpr int GEMV_BATCH = 4;  // chunks per prefetch batch (two batches in flight)
constexpr size_t GEMV_LDS_BUDGET = 65536;

// Stage groups [g0, g0 + GP) of M activation rows: XL[m][g - g0][j] = (x[32g+2j], x[32g+16+2j],
// x[32g+2j+1], x[32g+17+2j]) and GS[m][g - g0] = x[32g] + x[32g+1] + ... + x[32g+31] (W:22 order).
template <int MT>
__device__ __forceinline__ void stage_x(const GemvArgs& a, int M, int g0, int GP, float4* XL, float* GS) {
  for (int idx = threadIdx.x; idx < MT * GP * 8; idx += GEMV_THREADS) {
    const int j = idx & 7, g = (idx >> 3) % GP, m = idx / (GP * 8);
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (m < M) {
      const float* b = a.x + (size_t)m * a.ldx + (size_t)(g0 + g) * 32;
      v = make_float4(b[2 * j], b[16 + 2 * j], b[2 * j + 1], b[17 + 2 * j]);
    }
    XL[idx] = v;
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < MT * GP; idx += GEMV_THREADS) {
    const float4* q = XL + (size_t)idx * 8;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) s += (i & 1) ? q[i >> 1].z : q[i >> 1].x;
#pragma unroll
    for (int i = 0; i < 16; ++i) s += (i & 1) ? q[i >> 1].w : q[i >> 1].y;
    GS[idx] = s;
  }
  __syncthreads();
}

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
  const int GP = a.kphase / 32, CP = a.kphase / 256;  // groups / chunks per phase
  const int M = a.active ? min(a.M, *a.active) : a.M;  // rows beyond a device-side count are idle
  float4* XL = lds4;                                       // [MT][GP][8]
  float* GS = reinterpret_cast<float*>(lds4 + MT * GP * 8);  // [MT][GP]
  const bool one_phase = CP == GC;
  if (one_phase) stage_x<MT>(a, M, 0, GP, XL, GS);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 7, mslot = (lane >> 3) % MS, rslot = lane / LPR;
  const int m0 = mslot * MPL;
  // activation rows this lane reads, clamped into the staged [MT] rows (when MS * MPL > MT the
  // last lane group has slots past MT; their results are never stored)
  int mrow[MPL];
#pragma unroll
  for (int q = 0; q < MPL; ++q) mrow[q] = min(m0 + q, MT - 1);
  const int moff = min(m0 + (j < MPL ? j : MPL - 1), MT - 1);  // row of this lane's offset chain
  const int ntiles = a.tiles[3];
  float lrun = -INFINITY;  // EPI_SCREEN: running max of L for activation row j of this lane

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

    // chunk c (global), staged group index of its first group = gl
    auto chunk = [&](const uint4 wv, const uint4 sv, const int c, const int gl) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t d = k == 0 ? wv.x : (k == 1 ? wv.y : (k == 2 ? wv.z : wv.w));
        const uint32_t s2 = k == 0 ? sv.x : (k == 1 ? sv.y : (k == 2 ? sv.z : sv.w));
        const uint32_t lo = d & 0x0F0F0F0Fu, hi = (d >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int g = gl + 2 * k + h;
          const float l0 = (float)((lo >> (16 * h)) & 0xFFu);
          const float l1 = (float)((lo >> (16 * h + 8)) & 0xFFu);
          const float h0 = (float)((hi >> (16 * h)) & 0xFFu);
          const float h1 = (float)((hi >> (16 * h + 8)) & 0xFFu);
          const float sc = h ? as_f32(s2 & 0xFFFF0000u) : as_f32(s2 << 16);
#pragma unroll
          for (int q = 0; q < MPL; ++q) {
            const float4 xv = XL[(mrow[q] * GP + g) * 8 + j];
            float av = l0 * xv.x;
            av = fmaf(l1, xv.y, av);
            av = fmaf(h0, xv.z, av);
            av = fmaf(h1, xv.w, av);
            row[q] = fmaf(av, sc, row[q]);
          }
          off = fmaf(sc, GS[moff * GP + g], off);
        }
      }
      (void)c;
    };

    const uint4 z4 = make_uint4(0, 0, 0, 0);
    for (int p0 = 0; p0 < GC; p0 += CP) {  // phases of K
      if (!one_phase) stage_x<MT>(a, M, p0 * 8, GP, XL, GS);
      const int pend = p0 + CP;
      uint4 wA[GEMV_BATCH], sA[GEMV_BATCH], wB[GEMV_BATCH], sB[GEMV_BATCH];
#pragma unroll
      for (int b = 0; b < GEMV_BATCH; ++b) {
        const bool ok = valid && p0 + b < pend;
        wA[b] = ok ? wp[(size_t)(p0 + b) * 8] : z4;
        sA[b] = ok ? sp[p0 + b] : z4;
      }
      for (int c0 = p0; c0 < pend; c0 += 2 * GEMV_BATCH) {
#pragma unroll
        for (int b = 0; b < GEMV_BATCH; ++b) {  // batch B in flight while batch A is consumed
          const int c = c0 + GEMV_BATCH + b;
          const bool ok = valid && c < pend;
          wB[b] = ok ? wp[(size_t)c * 8] : z4;
          sB[b] = ok ? sp[c] : z4;
        }
#pragma unroll
        for (int b = 0; b < GEMV_BATCH; ++b)
          if (c0 + b < pend) chunk(wA[b], sA[b], c0 + b, (c0 + b - p0) * 8);
#pragma unroll
        for (int b = 0; b < GEMV_BATCH; ++b) {
          const int c = c0 + 2 * GEMV_BATCH + b;
          const bool ok = valid && c < pend;
          wA[b] = ok ? wp[(size_t)c * 8] : z4;
          sA[b] = ok ? sp[c] : z4;
        }
#pragma unroll
        for (int b = 0; b < GEMV_BATCH; ++b)
          if (c0 + GEMV_BATCH + b < pend) chunk(wB[b], sB[b], c0 + GEMV_BATCH + b, (c0 + GEMV_BATCH + b - p0) * 8);
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
      if (own) {
        const float cf = a.coef[n], hn = a.hn[m];
        lrun = fmaxf(lrun, fmaf(-cf, hn, y));
        a.y[0][(size_t)m * a.ldy[0] + n] = fmaf(cf, hn, y);
      }
    }
  }
  if (EPI == EPI_SCREEN) {
    // block max of L per activation row (max is order free); one partial per block, reduced
    // by the consumer instead of a same-address atomic per wave
    static_assert(EPI != EPI_SCREEN || MS == 1, "the screen runs one lane group per row");
    __shared__ float wl[GEMV_THREADS / 64][8];
#pragma unroll
    for (int sft = 8; sft < 64; sft <<= 1) lrun = fmaxf(lrun, __shfl_xor(lrun, sft, 64));  // same j = same m
    if (lane < 8) wl[wave][lane] = lrun;
    __syncthreads();
    if (threadIdx.x < MT) {
      float v = -INFINITY;
      for (int w = 0; w < GEMV_THREADS / 64; ++w) v = fmaxf(v, wl[w][threadIdx.x]);
      a.lpart[(size_t)threadIdx.x * gridDim.x + blockIdx.x] = v;
    }
  }
}

static size_t gemv_lds(int MT, int kphase) {
  const int GP = kphase / 32;
  return (size_t)MT * GP * 8 * sizeof(float4) + (size_t)MT * GP * sizeof(float);
}

template <int MT, int MS, int EPI>
static void launch_t(const GemvArgs& a, hipStream_t st, int grid) {
  const size_t lds = gemv_lds(MT, a.kphase);
  if (lds > 65536) {  // gfx950 gives a workgroup up to 160 KB of LDS on request
    static bool raised = false;
    if (!raised) {
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemv<MT, MS, EPI>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, 163840);
      raised = true;
    }
  }
  hipLaunchKernelGGL((k_gemv<MT, MS, EPI>), dim3(grid), dim3(GEMV_THREADS), lds, st, a);
}

template <int MT, int EPI>
static void launch_ms(const GemvArgs& a, int ms, hipStream_t st, int grid) {
  if constexpr (EPI != EPI_STORE) {  // fused epilogues pair rows inside a wave: one lane group per row
    (void)ms;
    launch_t<MT, 1, EPI>(a, st, grid);
  } else {
    switch (ms) {
      case 1: launch_t<MT, 1, EPI>(a, st, grid); break;
      case 2: if constexpr (MT >= 2) launch_t<MT, 2, EPI>(a, st, grid); break;
      case 4: if constexpr (MT >= 4) launch_t<MT, 4, EPI>(a, st, grid); break;
      default: if constexpr (MT >= 8) launch_t<MT, 8, EPI>(a, st, grid); break;
    }
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

// largest K phase (a multiple of 256 dividing K) whose staged activations fit the budget
static int pick_kphase(int MT, int K) {
  for (int parts = 1; parts <= K / 256; ++parts) {
    if (K % parts || (K / parts) % 256) continue;
    if (gemv_lds(MT, K / parts) <= GEMV_LDS_BUDGET) return K / parts;
  }
  return 256;
}

static int plan(GemvArgs& a, int epi) {
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
  a.kphase = pick_kphase(MT, a.K);
  return ms;
}

int gemv_grid(const GemvArgs& a_in, int epi, int grid_cap) {
  GemvArgs a = a_in;
  plan(a, epi);
  return (grid_cap > 0 && a.tiles[3] > grid_cap) ? grid_cap : a.tiles[3];
}

int launch_gemv(const GemvArgs& a_in, int epi, hipStream_t st, int grid_cap) {
  GemvArgs a = a_in;
  const int MT = a.M;
  const int ms = plan(a, epi);
  const int grid = (grid_cap > 0 && a.tiles[3] > grid_cap) ? grid_cap : a.tiles[3];
#define G4V_CASE(mt)                                                               \
  case mt:                                                                         \
    if (epi == EPI_STORE) launch_ms<mt, EPI_STORE>(a, ms, st, grid);               \
    else if (epi == EPI_GATEUP) launch_ms<mt, EPI_GATEUP>(a, ms, st, grid);        \
    else launch_ms<mt, EPI_SCREEN>(a, ms, st, grid);                               \
    break;
  switch (MT) {
    G4V_CASE(1) G4V_CASE(2) G4V_CASE(3) G4V_CASE(4) G4V_CASE(5) G4V_CASE(6) G4V_CASE(7) G4V_CASE(8)
    default: break;
  }
#undef G4V_CASE
  return grid;
}

}  // namespace g4v
