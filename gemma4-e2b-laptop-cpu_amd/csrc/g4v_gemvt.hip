// g4v_gemvt.hip -- row-tile W4G32 GEMV for the verify pass's skinny products, gfx950.
//
// Same arithmetic as k_gemv (g4v_gemv.hip), i.e. w4::gemm_rows_tile (engine/w4g32_avx2.h:64-96)
// bit for bit: chain lane j of output (n, m) runs
//   a = lo(b_j) xe_j; a = fma(lo(b_8+j), xe_8+j, a); a = fma(hi(b_j), xo_j, a);
//   a = fma(hi(b_8+j), xo_8+j, a); r_j = fma(a, sc_g, r_j);   off = fma(sc_g, gsum_g, off)
// over the groups g in order, and y = ((r0+r4)+(r1+r5))+((r2+r6)+(r3+r7)) - 8 off.
//
// The lane mapping is transposed: a thread holds one output row of one chain lane j for MPL
// activation rows, and the rows of a tile (TR = 64 or 32) are consecutive lanes, so the
// activation operand of every FMA is the same for the TR lanes of a chain lane (a broadcast
// LDS read per group and row) and a block of 8 TR threads (j = 0..7) finishes its TR rows with
// one LDS exchange.  A block stages only its own MPL activation rows, so even
// K = 6144 fits in one pass, and the launch has one block per (64-row tile, row subset): the
// blocks of a tile are placed on the same XCD (round-robin block order), whose L2 then serves
// the tile's weights to all of them.
#include "g4v_internal.h"

namespace g4v {


__constant__ uint64_t c_expf_tab_t[32] = G4V_EXPF_TABLE;
// chunks per weight batch (two batches in flight): 2 for three and four activation rows keeps
// the kernel within 4 waves per SIMD, i.e. two 512-thread blocks per CU
template <int MPL>
constexpr int gt_batch() { return MPL >= 3 ? 2 : 4; }

// re-laid wr[n][c][j] -> tw[n/64][c][j][n%64]; scales s[n][G] (uint4 = 8 groups) -> ts[n/64][c][n%64]
__global__ void k_tile_w4(const uint4* __restrict__ wr, const uint4* __restrict__ s4, uint4* __restrict__ tw,
                          uint4* __restrict__ ts, int N, int K) {
  const int GC = K / 256;
  const size_t total = (size_t)N * GC * 8;
  for (size_t u = (size_t)blockIdx.x * blockDim.x + threadIdx.x; u < total; u += (size_t)gridDim.x * blockDim.x) {
    const int j = (int)(u & 7);
    const size_t nc = u >> 3;
    const int c = (int)(nc % GC);
    const size_t n = nc / GC;
    tw[(((n >> 6) * GC + c) * 8 + j) * 64 + (n & 63)] = wr[u];
    if (j == 0) ts[((n >> 6) * GC + c) * 64 + (n & 63)] = s4[nc];
  }
}

void launch_tile_w4(const uint4* wr, const uint16_t* s, uint4* tw, uint4* ts, int N, int K, hipStream_t st) {
  const size_t total = (size_t)N * (K / 256) * 8;
  int grid = (int)((total + 255) / 256);
  if (grid > 65536) grid = 65536;
  hipLaunchKernelGGL(k_tile_w4, dim3(grid), dim3(256), 0, st, wr, reinterpret_cast<const uint4*>(s), tw, ts, N, K);
}

// gate / up pair: 64-row tile t holds, for pairs n = 32t .. 32t+31, rows [gate 16, up 16, gate 16,
// up 16]: gate n at local row 32 (i / 16) + i % 16 and up n at 16 more (i = n - 32t), so every
// 32-row half holds whole pairs (N each, N % 32 == 0)
__global__ void k_tile_w4_pair(const uint4* __restrict__ wg, const uint4* __restrict__ sg,
                               const uint4* __restrict__ wu, const uint4* __restrict__ su, uint4* __restrict__ tw,
                               uint4* __restrict__ ts, int N, int K) {
  const int GC = K / 256;
  const size_t total = (size_t)2 * N * GC * 8;
  for (size_t u = (size_t)blockIdx.x * blockDim.x + threadIdx.x; u < total; u += (size_t)gridDim.x * blockDim.x) {
    const int j = (int)(u & 7);
    const size_t nc = u >> 3;
    const int c = (int)(nc % GC);
    const size_t r = nc / GC;  // paired row: tile r / 64, local row r % 64
    const size_t t = r >> 6, lr = r & 63;
    const size_t n = t * 32 + (lr >> 5) * 16 + (lr & 15);
    const bool up = (lr & 16) != 0;
    const uint4 w = up ? wu[(n * GC + c) * 8 + j] : wg[(n * GC + c) * 8 + j];
    tw[((t * GC + c) * 8 + j) * 64 + lr] = w;
    if (j == 0) ts[(t * GC + c) * 64 + lr] = up ? su[n * GC + c] : sg[n * GC + c];
  }
}

void launch_tile_w4_pair(const uint4* wg, const uint16_t* sg, const uint4* wu, const uint16_t* su, uint4* tw,
                         uint4* ts, int N, int K, hipStream_t st) {
  const size_t total = (size_t)2 * N * (K / 256) * 8;
  int grid = (int)((total + 255) / 256);
  if (grid > 65536) grid = 65536;
  hipLaunchKernelGGL(k_tile_w4_pair, dim3(grid), dim3(256), 0, st, wg, reinterpret_cast<const uint4*>(sg), wu,
                     reinterpret_cast<const uint4*>(su), tw, ts, N, K);
}

struct GemvTDev {
  GemvTArgs a;
  int tiles[4];  // prefix sums of 64-row tiles per matrix
  int nsub;      // row subsets: block slot k -> subset k % nsub, tile group k / nsub
};

// LDS: activations [MPL][G][8 + 1] float4 (staged; a pad float4 after each group spreads the
// per-group accesses of the prologue over the banks), group sums [MPL][G], chain sums [MPL][8][64],
// offsets [MPL][64], outputs of the gate/up epilogue [MPL][64]; the norm prologue adds its two
// weight rows [2][H] and RMS factors [2][MPL]
static size_t gemvt_lds(int mpl, int K, bool nrm, int tr, bool mrg) {
  const int G = K / 32;
  return (size_t)mpl * G * 9 * 16 + (size_t)mpl * G * 4 + (size_t)mpl * 8 * tr * 4 + (size_t)mpl * tr * 4 * 2 +
         (mrg ? (size_t)mpl * NQ * (3 * MAXT + 1) * 4 : 0) +
         (nrm ? (size_t)2 * H * 4 + (size_t)2 * mpl * 4 : 0);
}

// MRG: the merge prologue (GemvTArgs::mrg_po), NRM: the norm prologue (GemvTArgs::nrm_mode);
// variants of their own so that their registers do not weigh on the other launches
// TR: rows per tile (64: a wave is 64 rows of one chain lane; 32: a wave is 32 rows of two
// chain lanes); a block is the TR x 8 (row, chain lane) pairs of one tile, 8 TR threads
// KT: the reduction length when fixed at compile time (0: a.K), so that the LDS addresses of the
// staged activations fold into instruction offsets
// XM: the Gemma per-layer-input gate (GemvTArgs::epi_pli; NRM prologue in mode 3)
// The arguments a block needs before its first loads lead the list (up to 16 dwords), so that
// they arrive preloaded in scalar registers at launch (kernel-argument preloading) instead of
// through a load of the argument segment: the prologue's four input pointers pa..pd (MRG: po, pm,
// pl; NRM: o, xin, w1, w2; otherwise xs, gs), matrix 0's tiles, and the geometry packed in two
// words -- gx = nsub | (MRG: T, NRM: nmode) << 8 | M << 16, tlp = tiles[1] | tiles[2] << 10 |
// tiles[3] << 20 (14 dwords: all that the launch preloads).
// The rest (matrices 1 and 2, the outputs, the epilogue's operands) comes from the argument
// block d, read while the prologue's loads are in flight.
template <int MPL, bool MRG, bool NRM, int TR, int KT = 0, int XM = 0>
__global__ __launch_bounds__(TR * 8) void k_gemv_t(const float* __restrict__ pa, const float* __restrict__ pb,
                                                   const float* __restrict__ pc, const float* __restrict__ pd,
                                                   const uint4* __restrict__ w0w, const uint4* __restrict__ w0s,
                                                   int gx, int tlp, GemvTDev d) {
  constexpr int NT = TR * 8;
  const GemvTArgs& a = d.a;
  const int nsub = gx & 0xFF, M = gx >> 16, tl1 = tlp & 0x3FF, tl2 = (tlp >> 10) & 0x3FF, tl3 = tlp >> 20;
  const int T = MRG ? (gx >> 8) & 0xFF : 0, nmode = NRM ? (gx >> 8) & 0xFF : 0;
  const int K = KT ? KT : a.K, G = K / 32, GC = K / 256;
  // block -> (tile, row subset); the tiles of XCD x (block % 8) are x, x + 8, ...
  const int xcd = blockIdx.x & 7, kq = blockIdx.x >> 3;
  const int sub = kq % nsub, t = (kq / nsub) * 8 + xcd;
  if (t >= tl3) return;
  const int m0 = sub * MPL;
  // thread -> (chain lane j, row lane of the tile); rows of a 32-row tile are one half of a
  // 64-row tile of the storage layout
  const int j = threadIdx.x / TR, lane = threadIdx.x % TR;
  extern __shared__ float4 lds4[];
  float4* XL = lds4;                                         // [MPL][G][8]
  float* GSL = reinterpret_cast<float*>(XL + MPL * G * 9);  // [MPL][G]
  // float4 u = (row * G + group) * 8 + k of the rows is held at pad(u)
  auto pad = [](int u) { return u + (u >> 3); };
  float* RL = GSL + MPL * G;                                 // [MPL][8][TR]
  float* OFL = RL + MPL * 8 * TR;                            // [MPL][TR]
  float* YL = OFL + MPL * TR;                                // [MPL][TR]

  const int mi = (t >= tl1) + (t >= tl2);
  const int tl = t - (mi == 0 ? 0 : (mi == 1 ? tl1 : tl2));
  const int t64 = tl / (64 / TR), r64 = (tl % (64 / TR)) * TR + lane;  // storage tile and row
  // the tiles of matrices 1 and 2 come from the argument block: chosen in weights_after, once the
  // prologue's loads are on their way
  const uint4 *wp = nullptr, *sp = nullptr;  // chunk c at wp + c * 512, sp + c * 64
  auto choose_mat = [&]() {
    const uint4* Ww = mi == 0 ? w0w : (mi == 1 ? a.mat[1].w : a.mat[2].w);
    const uint4* Ws = mi == 0 ? w0s : (mi == 1 ? a.mat[1].s : a.mat[2].s);
    wp = Ww + ((size_t)t64 * GC * 8 + j) * 64 + r64;
    sp = Ws + (size_t)t64 * GC * 64 + r64;
  };
  constexpr int GT_B = gt_batch<MPL>();
  uint4 wA[GT_B], sA[GT_B], wB[GT_B], sB[GT_B];
  auto load_batch = [&](uint4 (&w)[GT_B], uint4 (&s)[GT_B], int c0) {  // indices clamped
#pragma unroll
    for (int b = 0; b < GT_B; ++b) {
      const int c = min(c0 + b, GC - 1);
      w[b] = wp[(size_t)c * 512];
      s[b] = sp[(size_t)c * 64];
    }
  };
  // The prologue's own loads (activations, partials, residual rows) are issued first and the
  // first weight batch right after them: the load counter retires in issue order, so the
  // prologue then waits for its operands only, while the weights stream in behind it.
  // An execution barrier (no memory wait) first: every wave of the block has issued its prologue
  // loads before any wave's weights queue behind them in the CU's memory pipeline.
  auto weights_after = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    choose_mat();
    load_batch(wA, sA, 0);
    __builtin_amdgcn_sched_barrier(0);
  };

  // the block's activation rows m0 .. m0 + MPL - 1 (rows >= M staged as zeros, never stored)
  const int RW = G * 8;
  if constexpr (MRG) {
    // E:1019-1059 per (row, head h): M0 = max of max_t over the splits with l_t > 0,
    // sc_t = libm expf(max_t - M0), l = sum_t (double) l_t sc_t, inv = (float)(1 / l); then per
    // element y = r16((fma chain over those t of o_t sc_t) * inv).  Thread f < MPL * NQ forms
    // the factors of pair f once (SCL, -1 marks a split without positions); every thread then
    // runs the chains of its elements 4u .. 4u+3 (one head) and stores them staged.
    float* XF = reinterpret_cast<float*>(XL);
    float* SCL = YL + MPL * TR;            // [MPL][NQ][MAXT]
    float* INVL = SCL + MPL * NQ * MAXT;   // [MPL][NQ]
    constexpr int NI = MPL * (NQ * HD / 4) / NT;  // elements groups per thread (K = NQ * HD)
    constexpr int PT = 8;                         // splits whose partials are prefetched
    // thread f < MPL * NQ * MAXT takes split ft of pair fp (row, head): the factors of the
    // splits are formed in parallel, only the sum l runs over them in order
    const int f = threadIdx.x, fp = f / MAXT, ft = f % MAXT;
    float* PLL = INVL + MPL * NQ;           // [MPL][NQ][MAXT]
    float* PML = PLL + MPL * NQ * MAXT;     // [MPL][NQ][MAXT]
    // the expf table goes to LDS with the partials (no dependent constant-memory load per split)
    __shared__ uint64_t ETAB[32];
    const uint64_t etv = c_expf_tab_t[f & 31];
    float plv = 0.f, pmv = 0.f;
    if (f < MPL * NQ * MAXT && ft < T) {
      const int m = min(m0 + fp / NQ, M - 1), h = fp % NQ;
      const size_t kk = ((size_t)ft * M + m) * NQ + h;
      plv = pc[kk];
      pmv = pb[kk];
    }
    float4 po[NI][PT];
    auto po_load = [&](int tb) {
#pragma unroll
      for (int it = 0; it < NI; ++it) {
        const int idx = threadIdx.x + it * NT, q = idx / (K / 4), u = idx - q * (K / 4);
        const int m = min(m0 + q, M - 1), h = (4 * u) / HD, i = (4 * u) % HD;
#pragma unroll
        for (int k = 0; k < PT; ++k) {
          const int tt = tb + k;
          po[it][k] = tt < T ? *reinterpret_cast<const float4*>(pa + (((size_t)tt * M + m) * NQ + h) * HD + i)
                             : make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
    };
    po_load(0);
    weights_after();
    if (f < MPL * NQ * MAXT) {
      PLL[f] = plv;
      PML[f] = pmv;
    }
    if (f < 32) ETAB[f] = etv;
    __syncthreads();
    if (f < MPL * NQ * MAXT) {
      float M0 = -1e30f;  // (max is order free)
#pragma unroll
      for (int tt = 0; tt < MAXT; ++tt)
        if (tt < T && PLL[fp * MAXT + tt] > 0) M0 = (M0 < PML[fp * MAXT + tt]) ? PML[fp * MAXT + tt] : M0;
      SCL[f] = (ft < T && plv > 0) ? libm_expf_neg(pmv - M0, ETAB) : -1.f;
    }
    __syncthreads();
    if (f < MPL * NQ) {
      double l = 0;
#pragma unroll
      for (int tt = 0; tt < MAXT; ++tt) {
        const float sc = SCL[f * MAXT + tt];
        if (tt < T && sc >= 0.f) l = fma((double)PLL[f * MAXT + tt], (double)sc, l);
      }
      INVL[f] = (float)(1.0 / l);
    }
    __syncthreads();
    float4 acc[NI];
#pragma unroll
    for (int it = 0; it < NI; ++it) acc[it] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int tb = 0; tb < T; tb += PT) {
      if (tb) po_load(tb);
#pragma unroll
      for (int it = 0; it < NI; ++it) {
        const int idx = threadIdx.x + it * NT, q = idx / (K / 4), h = (4 * (idx - q * (K / 4))) / HD;
        const float* scp = SCL + (q * NQ + h) * MAXT + tb;
#pragma unroll
        for (int k = 0; k < PT; ++k) {
          const float sc = scp[k];
          if (tb + k < T && sc >= 0.f) {
            acc[it].x = fmaf(po[it][k].x, sc, acc[it].x);
            acc[it].y = fmaf(po[it][k].y, sc, acc[it].y);
            acc[it].z = fmaf(po[it][k].z, sc, acc[it].z);
            acc[it].w = fmaf(po[it][k].w, sc, acc[it].w);
          }
        }
      }
    }
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      const int idx = threadIdx.x + it * NT, q = idx / (K / 4), u = idx - q * (K / 4);
      const int h = (4 * u) / HD;
      const float inv = INVL[q * NQ + h];
      const bool live = m0 + q < M;
      const float yv[4] = {acc[it].x, acc[it].y, acc[it].z, acc[it].w};
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        const int si = staged_index(4 * u + cc);
        XF[pad(q * (K / 4) + (si >> 2)) * 4 + (si & 3)] = live ? r16(yv[cc] * inv) : 0.f;
      }
    }
  } else if constexpr (NRM) {
    // E:1358-1361 (mode 1) / E:1375-1378 with E:1390-1404 (mode 2, the per-layer-embedding
    // branch zero) for the block's rows.  Wave q forms row q in registers (6 float4 per lane)
    // without block barriers: x1 = r16(xin + r16((r16(o) * r1) * w1)), then xa from x1 and r2,
    // written to XL in plain order; XL is then permuted in place into the staged order, one
    // thread per (row, group).
    //
    constexpr int RW4 = H / 4, PER = RW4 / 64;
    static_assert(NT / 64 >= MPL, "a wave per activation row");
    const int wq = threadIdx.x >> 6, ln = threadIdx.x & 63;
    const bool rowwave = wq < MPL;            // uniform per wave
    const bool live = rowwave && m0 + wq < M;  // rows past M are staged as zeros
    const int mr = min(m0 + wq, M - 1);
    const float4* o4 = reinterpret_cast<const float4*>(pa) + (size_t)mr * RW4 + ln;
    const float4* x4 = reinterpret_cast<const float4*>(pb) + (size_t)mr * RW4 + ln;
    const float4* w14 = reinterpret_cast<const float4*>(pc) + ln;
    const float4* w24 = reinterpret_cast<const float4*>(pd) + ln;
    float4 ov[PER], xv[PER];
    if (rowwave) {
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        ov[k] = o4[64 * k];
        xv[k] = x4[64 * k];
      }
    }
    weights_after();
    if (rowwave) {
      float4* XR = XL + (size_t)wq * G * 9;  // row wq, plain order (padded)
      auto xl_at = [&](int k) -> float4& { const int u = ln + 64 * k; return XR[u + (u >> 3)]; };
      // E:326-345: lane t of the reference's ss_avx2 sums x[16 s + t]^2 in double over s in
      // order, and the 16 lane sums meet as a_l = (p_l + p_{l+4}) + (p_{l+8} + p_{l+12}),
      // ss = (a_0 + a_2) + (a_1 + a_3).  The wave writes its row into its XL region chain-major
      // (chain t at 100 t: the 96 values of one chain contiguous, rows of chains spread over the
      // banks), lanes 0..15 run the 16 chains, and the sums meet through data-parallel moves.
      float* CR = reinterpret_cast<float*>(XR);
      auto rms_row = [&](const float4 (&v)[PER]) -> float {
#pragma unroll
        for (int k = 0; k < PER; ++k) {
          const float f[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const int e = 4 * (ln + 64 * k) + c;  // element e: chain e % 16, step e / 16
            CR[(e & 15) * 100 + (e >> 4)] = f[c];
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        double part = 0;
        if (ln < 16) {
          const float4* ch = reinterpret_cast<const float4*>(CR + ln * 100);
#pragma unroll
          for (int i = 0; i < H / 64; ++i) {
            const float4 q = ch[i];
            const double d0 = (double)q.x, d1 = (double)q.y, d2 = (double)q.z, d3 = (double)q.w;
            part = fma(d0, d0, part);
            part = fma(d1, d1, part);
            part = fma(d2, d2, part);
            part = fma(d3, d3, part);
          }
        }
        const double b2 = part + shl_d<4>(part);  // lane l: p_l + p_{l+4}
        const double c2 = b2 + shl_d<8>(b2);      // lanes 0..3: a_l
        const double d2 = c2 + shl_d<2>(c2);      // lanes 0, 1: a_0 + a_2, a_1 + a_3
        const double e2 = d2 + shl_d<1>(d2);      // lane 0: ss
        const uint64_t u = as_u64(e2);
        const double ss = as_f64(((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), 0) << 32) |
                                 (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, 0));
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        return 1.0f / sqrtf((float)(ss / H) + 1e-6f);
      };
      const bool after_mlp = nmode == 2;
      const float scal = a.nrm_scalar;
      float4 w1[PER];
#pragma unroll
      for (int k = 0; k < PER; ++k) w1[k] = w14[64 * k];
      float4 os[PER];
#pragma unroll
      for (int k = 0; k < PER; ++k)
        os[k] = keep4(live, make_float4(r16(ov[k].x), r16(ov[k].y), r16(ov[k].z), r16(ov[k].w)));
      const float r1 = rms_row(os);
      float4 x1[PER];
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        const float4 o = os[k], w = w1[k], xr = xv[k];
        float4 v = make_float4(r16(xr.x + r16((o.x * r1) * w.x)), r16(xr.y + r16((o.y * r1) * w.y)),
                               r16(xr.z + r16((o.z * r1) * w.z)), r16(xr.w + r16((o.w * r1) * w.w)));
        if (after_mlp) v = make_float4(r16(v.x * scal), r16(v.y * scal), r16(v.z * scal), r16(v.w * scal));
        x1[k] = keep4(live, v);
        if (t == 0 && live) reinterpret_cast<float4*>(a.nrm_xout)[(size_t)(m0 + wq) * RW4 + ln + 64 * k] = x1[k];
      }
      if constexpr (XM == 1) {  // (mode 3: x1 itself is the product's input)
#pragma unroll
        for (int k = 0; k < PER; ++k) xl_at(k) = x1[k];
      } else {
        float4 w2[PER];
#pragma unroll
        for (int k = 0; k < PER; ++k) w2[k] = w24[64 * k];
        const float r2 = rms_row(x1);
#pragma unroll
        for (int k = 0; k < PER; ++k) {
          const float4 tv = x1[k], w = w2[k];
          float4 v = make_float4((tv.x * r2) * w.x, (tv.y * r2) * w.y, (tv.z * r2) * w.z, (tv.w * r2) * w.w);
          if (!after_mlp) v = make_float4(r16(v.x), r16(v.y), r16(v.z), r16(v.w));
          xl_at(k) = v;
        }
      }
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < MPL * G; idx += NT) {  // staged order + group sums
      float4* b4 = XL + (size_t)idx * 9;  // row q = idx / G, group g = idx % G: 8 float4 in plain order
      float4 r[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) r[i] = b4[i];
      float sum = 0.f;  // W:22 the group's sequential sum
#pragma unroll
      for (int i = 0; i < 8; ++i) sum = (((sum + r[i].x) + r[i].y) + r[i].z) + r[i].w;
      const float* v = reinterpret_cast<const float*>(r);
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) b4[jj] = make_float4(v[2 * jj], v[16 + 2 * jj], v[2 * jj + 1], v[17 + 2 * jj]);
      GSL[idx] = sum;
    }
  } else {
    // K <= 6144 (or the fixed K, up to 12288): at most MPL * K / 4 staged float4 and MPL * K / 32
    // group sums per block
    constexpr int KMX = KT > 6144 ? KT : 6144;
    constexpr int NX = (MPL * (KMX / 4) + NT - 1) / NT, NG = (MPL * (KMX / 32) + NT - 1) / NT;
    float4 xr[NX];
    float gr[NG];
#pragma unroll
    for (int k = 0; k < NX; ++k) {
      const int u = min((int)threadIdx.x + k * NT, MPL * RW - 1), q = u / RW;
      xr[k] = reinterpret_cast<const float4*>(pa)[(size_t)min(m0 + q, M - 1) * RW + (u - q * RW)];
    }
    if (pb) {
#pragma unroll
      for (int k = 0; k < NG; ++k) {
        const int idx = min((int)threadIdx.x + k * NT, MPL * G - 1), q = idx / G;
        gr[k] = pb[(size_t)min(m0 + q, M - 1) * G + (idx - q * G)];
      }
    }
    weights_after();
#pragma unroll
    for (int k = 0; k < NX; ++k) {
      const int u = threadIdx.x + k * NT;
      if (u < MPL * RW) XL[pad(u)] = keep4(m0 + u / RW < M, xr[k]);
    }
    if (pb) {  // (the group sums a.gs)
#pragma unroll
      for (int k = 0; k < NG; ++k) {
        const int idx = threadIdx.x + k * NT;
        if (idx < MPL * G) GSL[idx] = m0 + idx / G < M ? gr[k] : 0.f;
      }
    }
  }
  __syncthreads();
  if ((!pb || MRG) && !NRM) {  // W:22 each group's sequential sum, from the staged copy
    for (int idx = threadIdx.x; idx < MPL * G; idx += NT) {
      const float4* q4 = XL + (size_t)idx * 9;
      float4 v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = q4[i];
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) s += (i & 1) ? v[i >> 1].z : v[i >> 1].x;
#pragma unroll
      for (int i = 0; i < 16; ++i) s += (i & 1) ? v[i >> 1].w : v[i >> 1].y;
      GSL[idx] = s;
    }
    __syncthreads();
  }

  float row[MPL], off = 0.f;
#pragma unroll
  for (int q = 0; q < MPL; ++q) row[q] = 0.f;
  const int qo = j % MPL;  // this wave's offset chain: activation row m0 + j % MPL
  const float4* xw = XL + j;   // row q, group g: xw[(q * G + g) * 9], the same for the whole wave
  const float* gw = GSL + qo * G;
  // off is used from the waves j < MPL only (OFL below): with 64-row tiles a wave is one chain
  // lane, so the other waves run the chunks without the off chain (two copies of the loop, no
  // branch per group)
  auto chunk = [&](const uint4 wv, const uint4 sv, const int c, auto OFF) {
    constexpr bool with_off = decltype(OFF)::value;
    const float4 gs4[2] = {*reinterpret_cast<const float4*>(gw + c * 8),
                           *reinterpret_cast<const float4*>(gw + c * 8 + 4)};
    float4 xv[2][MPL];
#pragma unroll
    for (int q = 0; q < MPL; ++q) xv[0][q] = xw[(q * G + c * 8) * 9];
#pragma unroll
    for (int i = 0; i < 8; ++i) {  // group 8c + i: dword i/2 of the chunk, half i%2
      if (i + 1 < 8) {
#pragma unroll
        for (int q = 0; q < MPL; ++q) xv[(i + 1) & 1][q] = xw[(q * G + c * 8 + i + 1) * 9];
      }
      const int k = i >> 1, h = i & 1;
      const uint32_t dw = k == 0 ? wv.x : (k == 1 ? wv.y : (k == 2 ? wv.z : wv.w));
      const uint32_t s2 = k == 0 ? sv.x : (k == 1 ? sv.y : (k == 2 ? sv.z : sv.w));
      uint32_t lo = dw & 0x0F0F0F0Fu, hi = (dw >> 4) & 0x0F0F0F0Fu;
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
      if constexpr (with_off) {
        const float4 g4 = gs4[i >> 2];
        const int e = i & 3;
        off = fmaf(sc, e == 0 ? g4.x : (e == 1 ? g4.y : (e == 2 ? g4.z : g4.w)), off);
      }
    }
  };
  auto sweep = [&](auto OFF) {
    for (int cb = 0; cb < GC; cb += GT_B) {
      load_batch(wB, sB, cb + GT_B);  // next batch in flight while this one is used
#pragma unroll
      for (int b = 0; b < GT_B; ++b)
        if (cb + b < GC) chunk(wA[b], sA[b], cb + b, OFF);  // uniform condition
#pragma unroll
      for (int b = 0; b < GT_B; ++b) {
        wA[b] = wB[b];
        sA[b] = sB[b];
      }
    }
  };
  if (TR == 64 && __builtin_amdgcn_readfirstlane(j) >= MPL)  // uniform: a wave of one chain lane
    sweep(std::false_type{});
  else
    sweep(std::true_type{});

  // the 8 chain lanes of each (row, output) meet in LDS: ((r0+r4)+(r1+r5))+((r2+r6)+(r3+r7)) - 8 off
#pragma unroll
  for (int q = 0; q < MPL; ++q) RL[(q * 8 + j) * TR + lane] = row[q];
  if (j < MPL) OFL[j * TR + lane] = off;
  __syncthreads();
  if ((int)threadIdx.x < MPL * TR) {
    const int q = threadIdx.x / TR, rl = threadIdx.x % TR, m = m0 + q;
    const float* r = RL + q * 8 * TR + rl;
    const float y = (((r[0] + r[4 * TR]) + (r[TR] + r[5 * TR])) + ((r[2 * TR] + r[6 * TR]) + (r[3 * TR] + r[7 * TR]))) -
                    8.f * OFL[q * TR + rl];
    if constexpr (XM == 1) {  // E:421-427 g2 = r16(r16(gelu8(r16 y)) * r16(pli)), staged for the next product
      const int n = tl * TR + rl;
      if (m < M)
        a.y[0][(size_t)m * a.ldy[0] + staged_index(n)] =
            r16(r16(gelu8(r16(y))) * r16(a.epi_pli[(size_t)m * a.epi_pli_ld + n]));
    } else if (!a.gateup) {
      const int n = tl * TR + rl, np = ((a.yperm >> mi) & 1) ? head16_index(n) : n;
      if (m < M) a.y[mi][(size_t)m * a.ldy[mi] + np] = y;
    } else {
      YL[q * TR + rl] = y;
    }
  }
  if (a.gateup) {  // E:292-299 act = rbf8(rbf8(gelu8(rbf8 g)) * rbf8 u), written staged
    __syncthreads();
    if ((int)threadIdx.x < MPL * TR / 2) {
      // pair p of the tile: gate at local row 32 (p / 16) + p % 16, up 16 rows after it
      const int q = threadIdx.x / (TR / 2), p = threadIdx.x % (TR / 2), m = m0 + q;
      const int gl = (p >> 4) * 32 + (p & 15);
      const float g = YL[q * TR + gl], u = YL[q * TR + gl + 16];
      const float act = r16(r16(gelu8(r16(g))) * r16(u));
      if (m < M) a.y[0][(size_t)m * a.ldy[0] + staged_index(tl * (TR / 2) + p)] = act;
    }
  }
}

// One activation row, a product of the staged row (xs; group sums gs, or formed here) and one
// matrix, K = 2048 NX: the chains of k_gemv_t with their terms formed by eight waves.  A block
// takes 8 output rows; phase p covers chunks 8p .. 8p+7, and wave s < 8 forms the group terms
//   a = lo(b_j) xe_j; a = fma(lo(b_8+j), xe_8+j, a); a = fma(hi(b_j), xo_j, a); a = fma(hi(b_8+j), xo_8+j, a)
// of chunk 8p + s for the 8 rows x 8 chain lanes into LDS, with the groups' scales, while wave 8
// continues the chains of phase p - 1 from the other buffer: lane (j, r) row = fma(a, sc, row)
// over the phase's groups in order, and the row's off = fma(sc, gsum, off).  Every value and
// every rounding is k_gemv_t's (one row per block).
constexpr int GS_PG = 64;  // groups per phase (8 chunks)
static size_t gemvs_lds(int K) {
  const int G = K / 32;
  return (size_t)G * 9 * 16 + (size_t)G * 4 + (size_t)2 * GS_PG * 64 * 4 + (size_t)2 * GS_PG * 8 * 4 + 64 * 4 + 8 * 4 +
         64 * 16 + 576 * 4;
}
// NX = K / 2048: float4 of the row each of the first 512 threads stages, and phases
template <int NX>
__global__ __launch_bounds__(576) void k_gemv_s(const float4* __restrict__ xs, const float* __restrict__ gs,
                                                W4Tile mat, float* __restrict__ y) {
  constexpr int K = NX * 2048, G = K / 32, GC = K / 256;
  extern __shared__ float4 lds4[];
  float4* XL = lds4;                                    // staged row, float4 u at u + u / 8
  float* GSL = reinterpret_cast<float*>(XL + G * 9);  // [G]
  float* AL = GSL + G;                                  // [2][GS_PG][8 j][8 rows]
  float* SCL = AL + 2 * GS_PG * 64;                     // [2][GS_PG][8 rows]
  float* RL = SCL + 2 * GS_PG * 8;                      // [8 j][8 rows]
  float* OFL = RL + 64;                                 // [8 rows]
  float4* PADX = reinterpret_cast<float4*>(OFL + 8);    // [64]: the staging stores of wave 8
  float* PADG = reinterpret_cast<float*>(PADX + 64);    // [576]: the group-sum stores past G
  const int tid = threadIdx.x, s = tid >> 6, j = (tid >> 3) & 7, r = tid & 7;
  const int n0 = blockIdx.x * 8, t64 = n0 >> 6, r64 = (n0 & 63) + r;
  // The row's loads first, then this wave's chunk of every phase (8p + s), all in flight from the
  // start: loads retire in issue order, so the staging waits for the row alone, and the LDS-only
  // barriers below leave the weights in flight (phase p waits for its own words only).
  // Every wave issues the same loads (buffer loads; a thread with nothing to fetch reads past the
  // resource and gets zeros), so the waits count the same younger loads in every wave.
  constexpr uint32_t OOB = 0x7FFFFF00u;
  float4 xr[NX];
  float gr;
  {
    const __amdgpu_buffer_rsrc_t xrs = buf_rsrc(xs, (uint32_t)K * 4);
#pragma unroll
    for (int k = 0; k < NX; ++k) {
      const uint4 u = buf_load16(xrs, tid < 512 ? (uint32_t)(tid + 512 * k) * 16 : OOB);
      xr[k] = make_float4(as_f32(u.x), as_f32(u.y), as_f32(u.z), as_f32(u.w));
    }
    const __amdgpu_buffer_rsrc_t grs = buf_rsrc(gs, gs ? (uint32_t)G * 4 : 0u);
    gr = as_f32((uint32_t)__builtin_amdgcn_raw_buffer_load_b32(grs, tid < G ? tid * 4 : (int)OOB, 0, 0));
  }
  // (issue order: the row's loads before the weights, also through the IR passes)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  uint4 wv[NX], sv[NX];
  {
    // the tile's words: chunk c of row slot (j, r64) at 512 c + 64 j + r64, its scales at 64 c + r64
    const __amdgpu_buffer_rsrc_t wrs = buf_rsrc(mat.w + (size_t)t64 * GC * 512, (uint32_t)GC * 512 * 16);
    const __amdgpu_buffer_rsrc_t srs = buf_rsrc(mat.s + (size_t)t64 * GC * 64, (uint32_t)GC * 64 * 16);
#pragma unroll
    for (int p = 0; p < NX; ++p) {
      const int c = 8 * p + s;
      wv[p] = buf_load16(wrs, s < 8 ? (uint32_t)(512 * c + 64 * j + r64) * 16 : OOB);
      sv[p] = buf_load16(srs, s < 8 ? (uint32_t)(64 * c + r64) * 16 : OOB);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // the row into LDS: every thread stores (the threads past the row into the pads), so the row's
  // loads are used where they are issued and stay ahead of the weights
#pragma unroll
  for (int k = 0; k < NX; ++k) {
    const int u = tid + 512 * k;
    *(tid < 512 ? XL + u + (u >> 3) : PADX + (tid - 512)) = xr[k];
  }
  *(tid < G ? GSL + tid : PADG + tid) = gr;  // (without gs, the sums are formed below)
  lds_barrier();
  if (!gs) {  // W:22 each group's sequential sum, from the staged copy (G <= 384)
    if (const int g = tid; g < G) {
      const float4* q4 = XL + (size_t)g * 9;
      float4 v[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = q4[i];
      float sm = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) sm += (i & 1) ? v[i >> 1].z : v[i >> 1].x;
#pragma unroll
      for (int i = 0; i < 16; ++i) sm += (i & 1) ? v[i >> 1].w : v[i >> 1].y;
      GSL[g] = sm;
    }
    lds_barrier();
  }
  const float4* xw = XL + j;  // group g: xw[9 g]
  float row = 0.f, off = 0.f;
#pragma unroll
  for (int p = 0; p <= NX; ++p) {
    if (s < 8) {
      if (p < NX) {  // the terms of phase p
        const int c = 8 * p + s;
        float* al = AL + (p & 1) * GS_PG * 64;
        float* scl = SCL + (p & 1) * GS_PG * 8;
        const uint4 wA = wv[p < NX ? p : 0], sA = sv[p < NX ? p : 0];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int k = i >> 1, h = i & 1, g = 8 * c + i, gl = 8 * s + i;
          const uint32_t dw = k == 0 ? wA.x : (k == 1 ? wA.y : (k == 2 ? wA.z : wA.w));
          const uint32_t s2 = k == 0 ? sA.x : (k == 1 ? sA.y : (k == 2 ? sA.z : sA.w));
          uint32_t lo = dw & 0x0F0F0F0Fu, hi = (dw >> 4) & 0x0F0F0F0Fu;
          asm volatile("" : "+v"(lo), "+v"(hi));
          const float l0 = (float)((lo >> (16 * h)) & 0xFFu);
          const float l1 = (float)((lo >> (16 * h + 8)) & 0xFFu);
          const float h0 = (float)((hi >> (16 * h)) & 0xFFu);
          const float h1 = (float)((hi >> (16 * h + 8)) & 0xFFu);
          const float sc = h ? as_f32(s2 & 0xFFFF0000u) : as_f32(s2 << 16);
          const float4 x4 = xw[(size_t)g * 9];
          float av = l0 * x4.x;
          av = fmaf(l1, x4.y, av);
          av = fmaf(h0, x4.z, av);
          av = fmaf(h1, x4.w, av);
          al[(gl * 8 + j) * 8 + r] = av;
          if (j == 0) scl[gl * 8 + r] = sc;
        }
      }
    } else if (p >= 1) {  // wave 8: the chains of phase p - 1 (every lane runs its row's off chain)
      const float* al = AL + ((p - 1) & 1) * GS_PG * 64 + j * 8 + r;
      const float* scl = SCL + ((p - 1) & 1) * GS_PG * 8 + r;
      const float* gsp = GSL + GS_PG * (p - 1);
#pragma unroll 8
      for (int gl = 0; gl < GS_PG; ++gl) {
        const float sc = scl[gl * 8];
        row = fmaf(al[gl * 64], sc, row);
        off = fmaf(sc, gsp[gl], off);
      }
    }
    lds_barrier();
  }
  // the 8 chain lanes of each row meet: ((r0+r4)+(r1+r5))+((r2+r6)+(r3+r7)) - 8 off
  if (s == 8) {
    RL[j * 8 + r] = row;
    if (j == 0) OFL[r] = off;
  }
  lds_barrier();
  if (tid < 8) {
    const float* q = RL + tid;
    y[n0 + tid] = (((q[0] + q[32]) + (q[8] + q[40])) + ((q[16] + q[48]) + (q[24] + q[56]))) - 8.f * OFL[tid];
  }
}

// the leading (preloaded) arguments of a launch of k_gemv_t: see the kernel
struct GemvTLead {
  const float *pa, *pb, *pc, *pd;
  const uint4 *w0w, *w0s;
  int gx, tl;
};
static GemvTLead gemvt_lead(const GemvTDev& d) {
  const GemvTArgs& a = d.a;
  GemvTLead L{};
  int hi = 0;
  if (a.mrg_po) {
    L.pa = a.mrg_po;
    L.pb = a.mrg_pm;
    L.pc = a.mrg_pl;
    hi = a.mrg_T;
  } else if (a.nrm_mode) {
    L.pa = a.nrm_o;
    L.pb = a.nrm_xin;
    L.pc = a.nrm_w1;
    L.pd = a.nrm_w2;
    hi = a.nrm_mode;
  } else {
    L.pa = reinterpret_cast<const float*>(a.xs);
    L.pb = a.gs;
  }
  L.w0w = a.mat[0].w;
  L.w0s = a.mat[0].s;
  L.gx = d.nsub | (hi << 8) | (a.M << 16);
  L.tl = d.tiles[1] | (d.tiles[2] << 10) | (d.tiles[3] << 20);
  return L;
}

#define G4V_GEMVT_ARGS L.pa, L.pb, L.pc, L.pd, L.w0w, L.w0s, L.gx, L.tl, d
template <int MPL, int TR>
static void launch_mpl(const GemvTDev& d, hipStream_t st, int grid) {
  const size_t lds = gemvt_lds(MPL, d.a.K, d.a.nrm_mode != 0, TR, d.a.mrg_po != nullptr);
  const dim3 g(grid), b(TR * 8);
  const int K = d.a.K;
  const GemvTLead L = gemvt_lead(d);
  // the verify pass's shapes at their default tiles get a fixed K: q/k/v and gate/up (norm
  // prologue, K 1536), down (K 6144)
  if (d.a.mrg_po) {  // (a fixed K costs the merge variant registers: it stays generic)
    if constexpr (MPL <= 2) hipLaunchKernelGGL((k_gemv_t<MPL, true, false, TR>), g, b, lds, st, G4V_GEMVT_ARGS);
  } else if (d.a.epi_pli) {
    hipLaunchKernelGGL((k_gemv_t<MPL, false, true, TR, 0, 1>), g, b, lds, st, G4V_GEMVT_ARGS);
  } else if (d.a.nrm_mode) {
    if constexpr ((MPL == 2 || MPL == 4) && TR == 64) {
      if (K == 1536) {
        hipLaunchKernelGGL((k_gemv_t<MPL, false, true, TR, 1536>), g, b, lds, st, G4V_GEMVT_ARGS);
        return;
      }
    }
    hipLaunchKernelGGL((k_gemv_t<MPL, false, true, TR>), g, b, lds, st, G4V_GEMVT_ARGS);
  } else {
    if constexpr (MPL == 1 && TR == 64) {
      if (K == 6144) {
        hipLaunchKernelGGL((k_gemv_t<MPL, false, false, TR, 6144>), g, b, lds, st, G4V_GEMVT_ARGS);
        return;
      }
    }
    if constexpr (MPL == 1) {
      if (K == 12288) {  // the Gemma-4-E2B layout's wide down projections
        hipLaunchKernelGGL((k_gemv_t<MPL, false, false, TR, 12288>), g, b, lds, st, G4V_GEMVT_ARGS);
        return;
      }
    }
    if constexpr (MPL == 2 && TR == 64) {
      if (K == 1536) {
        hipLaunchKernelGGL((k_gemv_t<MPL, false, false, TR, 1536>), g, b, lds, st, G4V_GEMVT_ARGS);
        return;
      }
    }
    hipLaunchKernelGGL((k_gemv_t<MPL, false, false, TR>), g, b, lds, st, G4V_GEMVT_ARGS);
  }
}
#undef G4V_GEMVT_ARGS

// mpl: activation rows per block (1 to 4); tr: rows per tile (64 or 32)
int launch_gemv_t(const GemvTArgs& a, hipStream_t st, int mpl, int tr) {
  // one activation row of a plain product with K >= 1024: the chains' terms formed by 8 waves
  const int nx = a.K / 2048;
  if (a.M == 1 && !a.mrg_po && !a.nrm_mode && !a.gateup && !a.epi_pli && !a.yperm && a.xs && a.mat[0].N % 64 == 0 &&
      a.mat[1].N == 0 && a.mat[2].N == 0 && a.K % 2048 == 0 && (nx == 1 || nx == 2 || nx == 3 || nx == 6)) {
    const size_t lds = gemvs_lds(a.K);
    static bool raised = false;  // more than 64 KB for K >= 6144 (gfx950: up to 160 KB on request)
    if (!raised) {
      const void* fns[] = {reinterpret_cast<const void*>(&k_gemv_s<1>), reinterpret_cast<const void*>(&k_gemv_s<2>),
                           reinterpret_cast<const void*>(&k_gemv_s<3>), reinterpret_cast<const void*>(&k_gemv_s<6>)};
      for (const void* f : fns) (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 163840);
      raised = true;
    }
    const int grid = a.mat[0].N / 8;
    switch (nx) {
      case 1: hipLaunchKernelGGL(k_gemv_s<1>, dim3(grid), dim3(576), lds, st, a.xs, a.gs, a.mat[0], a.y[0]); break;
      case 2: hipLaunchKernelGGL(k_gemv_s<2>, dim3(grid), dim3(576), lds, st, a.xs, a.gs, a.mat[0], a.y[0]); break;
      case 3: hipLaunchKernelGGL(k_gemv_s<3>, dim3(grid), dim3(576), lds, st, a.xs, a.gs, a.mat[0], a.y[0]); break;
      default: hipLaunchKernelGGL(k_gemv_s<6>, dim3(grid), dim3(576), lds, st, a.xs, a.gs, a.mat[0], a.y[0]); break;
    }
    return grid;
  }
  // the prologue register staging holds K <= 6144, and K = 12288 for one activation row per block
  // without a prologue of its own
  if (a.K % 256 || (a.K > 6144 && !(a.K == 12288 && mpl == 1 && !a.nrm_mode && !a.mrg_po && !a.epi_pli)))
    return 0;
  if (tr != 32) tr = 64;
  if (mpl < 1) mpl = 1;
  if (mpl > 4) mpl = 4;
  if (a.mrg_po && mpl > 2) mpl = 2;  // the merge variant exists for one and two rows
  GemvTDev d{};
  d.a = a;
  d.tiles[0] = 0;
  for (int i = 0; i < 3; ++i) d.tiles[i + 1] = d.tiles[i] + (a.gateup && i ? 0 : a.mat[i].N * (a.gateup ? 2 : 1) / tr);
  const int T = d.tiles[3], tg = (T + 7) / 8;
  if (T >= 1024 || a.M > 0x7FFF || (a.mrg_po && a.mrg_T > 255)) return 0;  // the packed launch geometry
  d.nsub = (a.M + mpl - 1) / mpl;
  const int grid = 8 * tg * d.nsub;
  if (tr == 64) {
    switch (mpl) {
      case 1: launch_mpl<1, 64>(d, st, grid); break;
      case 2: launch_mpl<2, 64>(d, st, grid); break;
      case 3: launch_mpl<3, 64>(d, st, grid); break;
      default: launch_mpl<4, 64>(d, st, grid); break;
    }
  } else {
    switch (mpl) {
      case 1: launch_mpl<1, 32>(d, st, grid); break;
      case 2: launch_mpl<2, 32>(d, st, grid); break;
      case 3: launch_mpl<3, 32>(d, st, grid); break;
      default: launch_mpl<4, 32>(d, st, grid); break;
    }
  }
  return grid;
}

}  // namespace g4v
