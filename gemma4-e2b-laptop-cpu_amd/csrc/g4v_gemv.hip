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
constexpr int GEMV_BATCH = 8;  // weight chunks per prefetch batch (two batches in flight)
constexpr size_t GEMV_LDS_BUDGET = 65536;
constexpr int GEMV_MAXR = 3;   // staged float4 per thread and activation row: phases of <= 3072

// Stage groups [g0, g0 + GP) of M activation rows: XL[m][g - g0][j] = (x[32g+2j], x[32g+16+2j],
// x[32g+2j+1], x[32g+17+2j]) and GS[m][g - g0] = x[32g] + x[32g+1] + ... + x[32g+31] (W:22 order).
// From the staged layout a row's phase is one contiguous run: stage_issue loads the thread's
// share into registers (clamped, always in bounds) and stage_commit stores it to LDS, so a
// caller issues every load of its prologue before the first wait.  From the plain layout each
// float4 gathers four scalars (stage_plain).
template <int MT>
struct StageRegs {
  float4 x[MT][GEMV_MAXR];
  float gs[MT];
};

template <int MT>
__device__ __forceinline__ void stage_issue(const GemvArgs& a, int M, int g0, int GP, StageRegs<MT>& r) {
  const int G = a.K / 32, RW = GP * 8;
#pragma unroll
  for (int m = 0; m < MT; ++m) {
#pragma unroll
    for (int q = 0; q < GEMV_MAXR; ++q)
      r.x[m][q] = a.xs[((size_t)min(m, M - 1) * G + g0) * 8 + min((int)threadIdx.x + q * GEMV_THREADS, RW - 1)];
    if (a.gs) r.gs[m] = a.gs[(size_t)min(m, M - 1) * G + g0 + min((int)threadIdx.x, GP - 1)];
  }
}

// stores the registers; the group sums are formed in LDS when the producer gave none
template <int MT>
__device__ __forceinline__ void stage_commit(const GemvArgs& a, int M, int GP, const StageRegs<MT>& r, float4* XL,
                                             float* GS) {
  const int RW = GP * 8;
#pragma unroll
  for (int m = 0; m < MT; ++m) {
#pragma unroll
    for (int q = 0; q < GEMV_MAXR; ++q) {
      const int u = threadIdx.x + q * GEMV_THREADS;
      if (u < RW) XL[m * RW + u] = keep4(m < M, r.x[m][q]);
    }
    if (a.gs && (int)threadIdx.x < GP) GS[m * GP + threadIdx.x] = m < M ? r.gs[m] : 0.f;
  }
  __syncthreads();
  if (!a.gs) {
#pragma unroll
    for (int m = 0; m < MT; ++m)
      for (int g = threadIdx.x; g < GP; g += GEMV_THREADS) {
        const float4* q = XL + (size_t)(m * GP + g) * 8;
        float4 v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = q[i];  // all eight reads in flight, then the ordered sum
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) s += (i & 1) ? v[i >> 1].z : v[i >> 1].x;
#pragma unroll
        for (int i = 0; i < 16; ++i) s += (i & 1) ? v[i >> 1].w : v[i >> 1].y;
        GS[m * GP + g] = s;
      }
    __syncthreads();
  }
}

template <int MT>
__device__ __forceinline__ void stage_plain(const GemvArgs& a, int M, int g0, int GP, float4* XL, float* GS) {
  const int RW = GP * 8;
#pragma unroll
  for (int m = 0; m < MT; ++m)
    for (int u = threadIdx.x; u < RW; u += GEMV_THREADS) {
      const int j = u & 7;
      const float* b = a.x + (size_t)min(m, M - 1) * a.ldx + (size_t)(g0 + (u >> 3)) * 32;
      XL[m * RW + u] = keep4(m < M, make_float4(b[2 * j], b[16 + 2 * j], b[2 * j + 1], b[17 + 2 * j]));
    }
  __syncthreads();
#pragma unroll
  for (int m = 0; m < MT; ++m)
    for (int g = threadIdx.x; g < GP; g += GEMV_THREADS) {
      const float4* q = XL + (size_t)(m * GP + g) * 8;
      float4 v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = q[i];
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) s += (i & 1) ? v[i >> 1].z : v[i >> 1].x;
#pragma unroll
      for (int i = 0; i < 16; ++i) s += (i & 1) ? v[i >> 1].w : v[i >> 1].y;
      GS[m * GP + g] = s;
    }
  __syncthreads();
}

// MT: activation rows (template bound), MS: lane groups sharing one output row,
// EPI: epilogue, MP: K is staged in several phases (kphase < K; otherwise kphase == K).
// Lane index = (rowslot * MS + mslot) * 8 + j.
template <int MT, int MS, int EPI, bool MP>
__global__ __launch_bounds__(GEMV_THREADS) void k_gemv(GemvArgs a) {
  constexpr int MPL = (MT + MS - 1) / MS;  // activation rows per lane
  constexpr int LPR = 8 * MS;               // lanes per output row
  constexpr int RPW = 64 / LPR;             // output rows per wave
  constexpr int RPB = RPW * (GEMV_THREADS / 64);
  constexpr int B = GEMV_BATCH;
  if (a.active && *a.active == 0) return;
  extern __shared__ float4 lds4[];
  const int K = a.K, G = K / 32, GC = K / 256;
  const int GP = a.kphase / 32, CP = a.kphase / 256;  // groups / chunks per phase
  const int M = a.active ? min(a.M, *a.active) : a.M;  // rows beyond a device-side count are idle
  float4* XL = lds4;                                       // [MT][GP][8]
  float* GS = reinterpret_cast<float*>(lds4 + MT * GP * 8);  // [MT][GP]
  uint4* SC = reinterpret_cast<uint4*>(GS + MT * GP);        // [RPB][GC]: 8 bf16 scales per chunk
  constexpr bool one_phase = !MP;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 7, mslot = (lane >> 3) % MS, rslot = lane / LPR;
  const int m0 = mslot * MPL;
  // LDS offsets of the activation rows this lane reads, clamped into the staged [MT] rows
  // (when MS * MPL > MT the last lane group has slots past MT; their results are never stored)
  int xoff[MPL];
#pragma unroll
  for (int q = 0; q < MPL; ++q) xoff[q] = min(m0 + q, MT - 1) * GP * 8 + j;
  const int goff = min(m0 + (j < MPL ? j : MPL - 1), MT - 1) * GP;  // this lane's offset chain row
  const int ntiles = a.tiles[3];
  float lrun = -INFINITY;  // EPI_SCREEN: running max of L for activation row j of this lane

  // which matrix / output row this lane serves in tile t, and its weight stream (rows past N
  // read row 0 and are never stored); the scales go through LDS (scales_issue / scales_commit)
  int mi = 0, n = 0;
  bool valid = false;
  const uint4* wp = nullptr;
  auto tile_ptrs = [&](int t) {
    if (EPI == EPI_GATEUP) {
      // row slots alternate gate / up for the same n: slot 2p -> gate, 2p+1 -> up
      mi = rslot & 1;
      n = t * (RPB / 2) + wave * (RPW / 2) + (rslot >> 1);
    } else {
      mi = (t >= a.tiles[1]) + (t >= a.tiles[2]);
      n = (t - a.tiles[mi]) * RPB + wave * RPW + rslot;
    }
    const W4Dev W = mi == 0 ? a.mat[0] : (mi == 1 ? a.mat[1] : a.mat[2]);
    valid = t < ntiles && n < W.N;
    wp = W.wr + ((size_t)(valid ? n : 0) * GC) * 8 + j;
  };
  // the bf16 scales of the tile's RPB rows, staged in LDS once per tile (row slot = the
  // lane's wave * RPW + rslot; rows past N get zeros): entries u = slot * GC + c, at most
  // GEMV_SCR per thread, loaded by scales_issue and stored by scales_commit
  constexpr int GEMV_SCR = 3;  // RPB * GC <= 32 * 24
  const int myslot = wave * RPW + rslot;
  uint4 scv[GEMV_SCR];
  auto scales_issue = [&](int t) {
#pragma unroll
    for (int q = 0; q < GEMV_SCR; ++q) {
      const int u = min((int)threadIdx.x + q * GEMV_THREADS, RPB * GC - 1);
      const int slot = u / GC, c = u - slot * GC;
      int ms, ns;
      if (EPI == EPI_GATEUP) {
        ms = slot & 1;
        ns = t * (RPB / 2) + (slot >> 1);
      } else {
        ms = (t >= a.tiles[1]) + (t >= a.tiles[2]);
        ns = (t - a.tiles[ms]) * RPB + slot;
      }
      const W4Dev W = ms == 0 ? a.mat[0] : (ms == 1 ? a.mat[1] : a.mat[2]);
      const bool ok = t < ntiles && ns < W.N;
      scv[q] = keep4(ok, reinterpret_cast<const uint4*>(W.s + (size_t)(ok ? ns : 0) * G)[c]);
    }
  };
  auto scales_commit = [&]() {
#pragma unroll
    for (int q = 0; q < GEMV_SCR; ++q) {
      const int u = threadIdx.x + q * GEMV_THREADS;
      if (u < RPB * GC) SC[u] = scv[q];
    }
  };
  uint4 wA[B], wB[B];  // weight batch being consumed, batch in flight
  // chunks c0 .. c0+B-1, indices clamped to clast (the extra loads are never consumed)
  auto load_batch = [&](uint4 (&w)[B], int c0, int clast) {
#pragma unroll
    for (int b = 0; b < B; ++b) w[b] = wp[(size_t)min(c0 + b, clast) * 8];
  };

  float row[MPL], off;
  // one chunk: 8 groups starting at staged group gl; the activation float4s of group g + 1
  // are read from LDS while group g is computed
  auto chunk = [&](const uint4 wv, const int c, const int gl) {
    const uint4 sv = SC[myslot * GC + c];
    const float4 gs4[2] = {*reinterpret_cast<const float4*>(GS + goff + gl),
                           *reinterpret_cast<const float4*>(GS + goff + gl + 4)};
    float4 xv[2][MPL];
#pragma unroll
    for (int q = 0; q < MPL; ++q) xv[0][q] = XL[xoff[q] + gl * 8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {  // group gl + i: dword i/2 of the chunk, half i%2
      if (i + 1 < 8) {
#pragma unroll
        for (int q = 0; q < MPL; ++q) xv[(i + 1) & 1][q] = XL[xoff[q] + (gl + i + 1) * 8];
      }
      const int k = i >> 1, h = i & 1;
      const uint32_t d = k == 0 ? wv.x : (k == 1 ? wv.y : (k == 2 ? wv.z : wv.w));
      const uint32_t s2 = k == 0 ? sv.x : (k == 1 ? sv.y : (k == 2 ? sv.z : sv.w));
      uint32_t lo = d & 0x0F0F0F0Fu, hi = (d >> 4) & 0x0F0F0F0Fu;
      // keep the two masked words: each nibble then converts with one byte-select convert
      // instead of a bit-field extract plus a convert
      asm volatile("" : "+v"(lo), "+v"(hi));
      const float l0 = (float)((lo >> (16 * h)) & 0xFFu);
      const float l1 = (float)((lo >> (16 * h + 8)) & 0xFFu);
      const float h0 = (float)((hi >> (16 * h)) & 0xFFu);
      const float h1 = (float)((hi >> (16 * h + 8)) & 0xFFu);
      const float sc = h ? as_f32(s2 & 0xFFFF0000u) : as_f32(s2 << 16);
#pragma unroll
      for (int q = 0; q < MPL; ++q) {
        const float4 x4 = xv[i & 1][q];
        float av = l0 * x4.x;
        av = fmaf(l1, x4.y, av);
        av = fmaf(h0, x4.z, av);
        av = fmaf(h1, x4.w, av);
        row[q] = fmaf(av, sc, row[q]);
      }
      const float4 g4 = gs4[i >> 2];
      const int e = i & 3;
      off = fmaf(sc, e == 0 ? g4.x : (e == 1 ? g4.y : (e == 2 ? g4.z : g4.w)), off);
    }
  };

  // every global load of the prologue (first weight batch, scales, activations, group sums)
  // is issued before the first wait
  tile_ptrs(blockIdx.x);
  load_batch(wA, 0, CP - 1);
  scales_issue(blockIdx.x);
  if (a.xs) {
    StageRegs<MT> sr;
    stage_issue<MT>(a, M, 0, GP, sr);
    scales_commit();
    stage_commit<MT>(a, M, GP, sr, XL, GS);
  } else {
    scales_commit();
    stage_plain<MT>(a, M, 0, GP, XL, GS);
  }
  bool have_A = true;

  for (int t = blockIdx.x; t < ntiles; t += gridDim.x) {
    tile_ptrs(t);
    if (t != (int)blockIdx.x) {  // later tiles of a grid-stride block: restage the scales
      scales_issue(t);
      __syncthreads();
      scales_commit();
      __syncthreads();
    }
#pragma unroll
    for (int q = 0; q < MPL; ++q) row[q] = 0.f;
    off = 0.f;
    for (int p0 = 0; p0 < GC; p0 += CP) {  // phases of K
      const int pend = p0 + CP;
      if (!have_A) {
        load_batch(wA, p0, pend - 1);  // in flight across the restaging below
        if (!one_phase) {
          if (a.xs) {
            StageRegs<MT> sr;
            stage_issue<MT>(a, M, p0 * 8, GP, sr);
            __syncthreads();  // every wave is done reading the previous phase's activations
            stage_commit<MT>(a, M, GP, sr, XL, GS);
          } else {
            __syncthreads();
            stage_plain<MT>(a, M, p0 * 8, GP, XL, GS);
          }
        }
      }
      have_A = false;
      for (int cb = p0; cb < pend; cb += B) {
        const bool more = cb + B < pend;             // (uniform)
        if (more) load_batch(wB, cb + B, pend - 1);  // next batch in flight while this one is used
#pragma unroll
        for (int b = 0; b < B; ++b)
          if (cb + b < pend) chunk(wA[b], cb + b, (cb + b - p0) * 8);  // uniform condition
        if (more) {
#pragma unroll
          for (int b = 0; b < B; ++b) wA[b] = wB[b];
        }
      }
    }
    // 8-lane tree sum per activation row; lane j keeps the sum of row m0 + j
    float mine = 0.f;
#pragma unroll
    for (int q = 0; q < MPL; ++q) {
      const float v = hsum8_lanes(row[q]);
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
      if (own && mi == 0) {
        const float act = r16(r16(gelu8(r16(y))) * r16(u));
        a.y[0][(size_t)m * a.ldy[0] + (a.y_staged ? staged_index(n) : n)] = act;
      }
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

// rows per 256-thread block for a given lane split
static inline int rows_per_block(int ms) { return (64 / (8 * ms)) * (GEMV_THREADS / 64); }

// activations [MT][GP][8] float4, group sums [MT][GP], scales of the tile's rows [rpb][K/256] uint4
static size_t gemv_lds(int MT, int kphase, int K, int rpb) {
  const int GP = kphase / 32;
  return (size_t)MT * GP * 8 * sizeof(float4) + (size_t)MT * GP * sizeof(float) + (size_t)rpb * (K / 256) * 16;
}

template <int MT, int MS, int EPI, bool MP>
static void launch_mp(const GemvArgs& a, hipStream_t st, int grid) {
  const size_t lds = gemv_lds(MT, a.kphase, a.K, rows_per_block(MS));
  if (lds > 65536) {  // gfx950 gives a workgroup up to 160 KB of LDS on request
    static bool raised = false;
    if (!raised) {
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemv<MT, MS, EPI, MP>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, 163840);
      raised = true;
    }
  }
  hipLaunchKernelGGL((k_gemv<MT, MS, EPI, MP>), dim3(grid), dim3(GEMV_THREADS), lds, st, a);
}

// multi-phase staging only exists for the plain-store epilogue (the fused epilogues run
// K = 1536 in one phase)
template <int MT, int MS, int EPI>
static void launch_t(const GemvArgs& a, hipStream_t st, int grid) {
  if constexpr (EPI == EPI_STORE) {
    if (a.kphase < a.K) {
      launch_mp<MT, MS, EPI, true>(a, st, grid);
      return;
    }
  }
  launch_mp<MT, MS, EPI, false>(a, st, grid);
}

template <int MT, int EPI>
static void launch_ms(const GemvArgs& a, int ms, hipStream_t st, int grid) {
  if constexpr (EPI == EPI_SCREEN) {  // the screen's block max runs one lane group per row
    (void)ms;
    launch_t<MT, 1, EPI>(a, st, grid);
  } else if constexpr (EPI == EPI_GATEUP) {  // gate / up row pairs need an even rows-per-wave count
    if (ms >= 2) {
      if constexpr (MT >= 2) launch_t<MT, 2, EPI>(a, st, grid);
    } else {
      launch_t<MT, 1, EPI>(a, st, grid);
    }
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


// Pick the lane split: spread activation rows over more lanes while the launch has
// fewer chain lanes than the GPU has SIMD lanes.
static int pick_ms(int MT, int Ntot, int epi) {
  if (epi == EPI_SCREEN) return 1;
  if (epi == EPI_GATEUP) return 1;
  int ms = 1;
  while (ms < 8 && ms * 2 <= MT && (long)Ntot * 8 * ms < 256L * 64 * 4) ms *= 2;
  return ms;
}

// largest K phase (a multiple of 256 dividing K) whose staged activations fit the budget
static int pick_kphase(int MT, int K, int rpb, size_t budget) {
  for (int parts = 1; parts <= K / 256; ++parts) {
    if (K % parts || (K / parts) % 256 || K / parts > GEMV_MAXR * GEMV_THREADS * 4) continue;
    if (gemv_lds(MT, K / parts, K, rpb) <= budget) return K / parts;
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
  size_t budget = a.lds_budget > 0 ? (size_t)a.lds_budget : GEMV_LDS_BUDGET;
  if (budget > 163840) budget = 163840;
  a.kphase = pick_kphase(MT, a.K, rpb, budget);
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
