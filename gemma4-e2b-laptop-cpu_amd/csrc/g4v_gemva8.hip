// g4v_gemva8.hip -- W4A8 products of a verify pass (M <= 8 activation rows) for gfx950.
//
// lin_multi with G_I8_ACTIVE (E:310-317) over decode rows: quant (engine/w4a8_avx2.h:30-42) of
// every activation row, then tile<MT> (engine/w4a8_avx2.h:46-61).  Per output (m, n):
//   a32[g] = sum_i u[n][32g+i] q[m][32g+i] - 8 sum[m][g]            (exact integer)
//   row    = fma((float)a32[g], sw[n][g] * sx[m][g], row)             over the groups g in order
// with sx = amax / 127, inv = sx > 0 ? 1 / sx : 0, q = RNE(x * inv), sum = sum of the q of the
// group (the same restatement as g4v_w4a8.hip, whose header shows that q never saturates).
//
// The group dots run on the matrix cores, one v_mfma_i32_16x16x32_i8 per (group, 16 outputs):
// A the quantised rows (rows >= M zero), B the weight nibbles as the signed bytes u - 8, so that
// D = sum_i q_i (u_i - 8) = a32 with no correction term (q unsaturated, every product and partial
// sum an integer far below 2^31); D is stored as float (|a32| < 2^24, exact).  Lane (m, n) then
// runs its chain over the groups in order on the VALU.
//
// The operand words: word h of (row m, group g) holds elements 8h + (0, 2, 4, 6, 1, 3, 5, 7) as
// int8, the order of the weight nibbles in a8 tiles (low nibbles, then high nibbles, of the
// group's bytes 4h .. 4h+3).
//
// Kernels, one launch per product of the fused verify pass:
//   k_gemv_a8p       a product of staged rows (o, down, the per-layer projection): a block per
//                    16 outputs walks K in phases of PG groups, quantises the phase's groups of
//                    every row into LDS, the next phase's weight words and row floats in flight
//                    while the current one is multiplied and chained; with PQ it copies instead
//                    the operand words that the rows' producer wrote (the split-KV merges for o,
//                    the gate / up blocks for down: a8_quant_group on the same floats);
//   k_gemv_a8n       a product whose prologue forms its rows as k_gemv_t's norm prologue does
//                    (q/k/v, gate/up, the per-layer-input gate; K = 1536, one phase) and
//                    quantises them in LDS; epilogues: y, the gate / up activation (staged; four
//                    tiles a block, each block one 32-group of every row, also quantised for down)
//                    or the per-layer-input gate (staged).
#include "g4v_internal.h"

namespace g4v {

typedef int i32x4_t __attribute__((ext_vector_type(4)));

// the B operand of one group: the lane's dword of weight nibbles (elements 8h .. 8h+7 of its
// output row) as the eight signed bytes u - 8, low nibbles first
__device__ __forceinline__ long a8_wbytes(uint32_t d) {
  uint32_t lo = (d & 0x0F0F0F0Fu) ^ 0x08080808u, hi = ((d >> 4) & 0x0F0F0F0Fu) ^ 0x08080808u;
  // a byte t = u ^ 8 holds u - 8 where u >= 8; where u < 8 (bit 3 of t set) u - 8 = t - 16: set
  // the high nibble
  lo |= (lo & 0x08080808u) * 0x1Eu;
  hi |= (hi & 0x08080808u) * 0x1Eu;
  return (long)((uint64_t)lo | ((uint64_t)hi << 32));
}

__device__ __forceinline__ float a8_scale(uint4 s4, int e) {  // bf16 scale e of a word of 8
  const uint32_t s2 = (e >> 1) == 0 ? s4.x : ((e >> 1) == 1 ? s4.y : ((e >> 1) == 2 ? s4.z : s4.w));
  return as_f32((e & 1) ? (s2 & 0xFFFF0000u) : (s2 << 16));
}

// ---- a product of quantised rows ----
// Block: the 16 outputs of one a8 tile (tiles of up to three matrices, in order), 512 threads in
// two roles.  K runs in phases of PG groups:
//   - every weight word of the block is requested at the start (at most A8P_NPM phases), so
//     the phases wait on one memory latency, not one each;
//   - waves 2-7 quantise the phase's groups of every row into LDS (a task per (group, row), the
//     rows padded to 2, 4 or 8; at most two tasks a thread, their floats fetched during the
//     previous phase) and stage the tile's scales;
//   - all eight waves multiply the phase's chunks (4 groups) w + 8k, k < NU, on the matrix cores
//     and store each (row, output, group)'s a32 as float, chain-major (rows past M are not
//     stored);
//   - waves 0-1 (a lane per (row, output)) run the phase's chain, forming sw * sx from the
//     staged scales as they go, while waves 2-7 quantise the next phase (PQ: copy its operand
//     words and row scales, fetched during the previous phase).
// The block's LDS traffic bounds the phases (a CU's LDS moves about 128 bytes a cycle): the
// chain reads 16-byte words of 4 groups, and only the matrix-core results go through LDS.
// One LDS barrier after the quantisation, one after the products (the weight words stay in
// flight across them).
// LDS: A32 [128][PG + 4] float (the chains' a32; the row stride puts a quarter wave's 16-byte
// reads on distinct banks), SXT [2][8][PG + 4] float (row scales) and SWL [2][PG / 8][16] uint4
// (weight scales), both by phase parity (the chain of a phase reads them while the next phase's
// are staged), AQL [PG][A8P_QS] operand words (word h of row m at 8 h + m; the group stride of 36
// spreads a wave's quantisation stores of 16 groups over the banks)
constexpr int A8P_PG = 64, A8P_NPM = 6;  // K <= 32 * 64 * 6 = 12288
constexpr int A8P_QS = 36;                // operand words per group in LDS (32 + padding)
template <int PG>
constexpr size_t a8p_lds() {
  return (size_t)128 * (PG + 4) * 4 + (size_t)2 * 8 * (PG + 4) * 4 + (size_t)2 * (PG / 8) * 16 * 16 +
         (size_t)PG * A8P_QS * 8;
}
template <int PG, bool PQ>
__global__ __launch_bounds__(512) void k_gemv_a8p(GemvTArgs a) {
  constexpr int PC = PG / 4, NU = PC / 8, S = PG + 4, QT = 384, QR = (PG * 8 + QT - 1) / QT;
  static_assert(PC % 8 == 0 && 2 * PG <= QT && QR <= 2, "whole chunks per wave; a scale word per staging thread");
  extern __shared__ float4 lds4[];
  float* A32 = reinterpret_cast<float*>(lds4);
  float* SXT = A32 + 128 * S;
  uint4* SWL = reinterpret_cast<uint4*>(SXT + 2 * 8 * S);
  uint64_t* AQL = reinterpret_cast<uint64_t*>(SWL + 2 * (PG / 8) * 16);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int M = a.M, K = a.K, G = K / 32, GC4 = G / 4, G8 = G / 8, nph = (G + PG - 1) / PG;
  const int t = blockIdx.x, tl1 = a.mat[0].N / 16, tl2 = tl1 + a.mat[1].N / 16;
  const int j = (t >= tl1) + (t >= tl2), mt = t - (j == 0 ? 0 : (j == 1 ? tl1 : tl2));
  const uint4* wp = (j == 0 ? a.mat[0].w : (j == 1 ? a.mat[1].w : a.mat[2].w)) + (size_t)mt * GC4 * 64 + lane;
  const uint4* sp = (j == 0 ? a.mat[0].s : (j == 1 ? a.mat[1].s : a.mat[2].s)) + (size_t)mt * G8 * 16;
  const int ar = lane & 15, ah = lane >> 4;
  const bool producer = w >= 2;  // (uniform per wave)
  const int tq = tid - 128;
  const int msh = M <= 2 ? 1 : (M <= 4 ? 2 : 3);

  // the staged floats of a producer's tasks (k = tq + QT r: group k >> msh of the phase, row
  // k & (2^msh - 1)); float4 jj of a group holds elements 2jj, 16 + 2jj, 2jj + 1, 17 + 2jj.  A task
  // past the rows or the groups reads zeros (offset past the resource).
  // PQ (rows quantised by their producer): a task fetches its group's four operand words and
  // scale instead (a8_quant_group's output for the same floats)
  const __amdgpu_buffer_rsrc_t xrs =
      PQ ? buf_rsrc(a.xq, (uint32_t)M * G * 32) : buf_rsrc(a.xs, (uint32_t)M * K * 4);
  const __amdgpu_buffer_rsrc_t xsr = buf_rsrc(a.xqs, PQ ? (uint32_t)M * G * 4 : 0u);
  constexpr int XW = PQ ? 2 : 8;  // 16-byte words a task fetches
  float4 xr[QR][XW];
  float xsv[QR];
  auto issue_x = [&](int p) {
#pragma unroll
    for (int r = 0; r < QR; ++r) {
      const int k = tq + QT * r, g = p * PG + (k >> msh), m = k & ((1 << msh) - 1);
      const bool ok = tq >= 0 && k < (PG << msh) && m < M && g < G;
      const uint32_t off = ok ? (PQ ? ((uint32_t)m * G + g) * 32u : ((uint32_t)m * K + 32u * g) * 4u) : 0x7FFFFF00u;
#pragma unroll
      for (int jj = 0; jj < XW; ++jj) {
        const uint4 u = buf_load16(xrs, off + 16 * jj);
        xr[r][jj] = make_float4(as_f32(u.x), as_f32(u.y), as_f32(u.z), as_f32(u.w));
      }
      if constexpr (PQ)
        xsv[r] = as_f32((uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
            xsr, ok ? (int)(((uint32_t)m * G + g) * 4u) : 0x7FFFFF00, 0, 0));
    }
  };
  // the phase's weight scales (producer thread tq < 2 PG: a word of the tile's scales; other
  // threads read zeros)
  const __amdgpu_buffer_rsrc_t srs = buf_rsrc(sp, (uint32_t)G8 * 16 * 16);
  uint4 stg;
  auto issue_s = [&](int p) {
    const int c8 = p * (PG / 8) + (tq >> 4);
    const bool ok = tq >= 0 && tq < 2 * PG && c8 < G8;
    stg = buf_load16(srs, ok ? ((uint32_t)c8 * 16 + (tq & 15)) * 16 : 0x7FFFFF00u);
  };
  // quant (engine/w4a8_avx2.h:33-41) of the producer's tasks into their operand words; rows
  // past M (and groups past G) get zeros
  auto quant = [&](int p) {
#pragma unroll
    for (int r = 0; r < QR; ++r) {
      const int k = tq + QT * r, gl = k >> msh, m = k & ((1 << msh) - 1);
      if (k < (PG << msh)) {
        uint64_t aq[4];
        float sx;
        if constexpr (PQ) {
#pragma unroll
          for (int h = 0; h < 4; ++h) {
            const float4 f = xr[r][h >> 1];
            aq[h] = (h & 1) ? ((uint64_t)__float_as_uint(f.w) << 32 | __float_as_uint(f.z))
                            : ((uint64_t)__float_as_uint(f.y) << 32 | __float_as_uint(f.x));
          }
          sx = xsv[r];
        } else {
          float v[32];
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) {
            v[2 * jj] = xr[r][jj].x;
            v[16 + 2 * jj] = xr[r][jj].y;
            v[2 * jj + 1] = xr[r][jj].z;
            v[17 + 2 * jj] = xr[r][jj].w;
          }
          sx = a8_quant_group(v, aq);
        }
        if (m >= M || p * PG + gl >= G) {
          sx = 0.f;
#pragma unroll
          for (int h = 0; h < 4; ++h) aq[h] = 0;
        }
        SXT[((p & 1) * 8 + m) * S + gl] = sx;
#pragma unroll
        for (int h = 0; h < 4; ++h) AQL[gl * A8P_QS + h * 8 + m] = aq[h];
      }
    }
    if (tq < 2 * PG) SWL[(p & 1) * (PG / 8) * 16 + tq] = stg;
  };

  // The first phase's floats first, then every phase's weight words of this wave's chunks
  // (chunks past the matrix read zeros): loads complete in issue order, so the first
  // quantisation waits for its floats alone.  Every wave issues the same loads (the chain
  // waves' row and scale loads read past their resources): the waits on the weight words then
  // count the same younger loads in both roles.
  issue_x(0);
  issue_s(0);
  const __amdgpu_buffer_rsrc_t wrs = buf_rsrc(wp - lane, (uint32_t)GC4 * 64 * 16);
  uint4 wq[A8P_NPM][NU];
#pragma unroll
  for (int p = 0; p < A8P_NPM; ++p)
#pragma unroll
    for (int k = 0; k < NU; ++k) {
      const int c = p * PC + w + 8 * k;
      wq[p][k] = buf_load16(wrs, c < GC4 ? ((uint32_t)c * 64 + lane) * 16 : 0x7FFFFF00u);
    }
  if (producer) quant(0);
  if (nph > 1) {
    issue_x(1);
    issue_s(1);
  }
  const int cm = (tid >> 4) & 7, cn = tid & 15;
  const bool chain = tid < 128 && cm < M;
  float acc = 0.f;
#pragma unroll
  for (int p = 0; p < A8P_NPM; ++p) {
    if (p >= nph) break;  // (uniform)
    const int gb = p * PG, ng = min(PG, G - gb);
    lds_barrier();  // the phase's operand words, row scales and weight scales are staged; A32 is free
    // the group dots of this wave's chunks: every operand read first, then the eight independent
    // products, then one 16-byte store per row and chunk (groups past G hold zero operand words
    // and are never chained)
    {
      uint64_t qw[NU][4];
#pragma unroll
      for (int k = 0; k < NU; ++k)
#pragma unroll
        for (int i = 0; i < 4; ++i) qw[k][i] = AQL[(4 * (w + 8 * k) + i) * A8P_QS + ah * 8 + (ar & 7)];  // word ah of row ar
      i32x4_t D[NU][4];
#pragma unroll
      for (int k = 0; k < NU; ++k) {
        const uint4 wv = wq[p][k];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t d = i == 0 ? wv.x : (i == 1 ? wv.y : (i == 2 ? wv.z : wv.w));
          D[k][i] = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)(ar < 8 ? qw[k][i] : 0), a8_wbytes(d),
                                                         i32x4_t{0, 0, 0, 0}, 0, 0, 0);  // rows >= 8 zero
        }
      }
      if (ah < 2 && 4 * ah < M) {  // rows 4 ah .. 4 ah + 3 of output ar
#pragma unroll
        for (int k = 0; k < NU; ++k)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            *reinterpret_cast<float4*>(A32 + ((4 * ah + r) * 16 + ar) * S + 4 * (w + 8 * k)) =
                make_float4((float)D[k][0][r], (float)D[k][1][r], (float)D[k][2][r], (float)D[k][3][r]);
      }
    }
    lds_barrier();
    if (!producer) {
      // the chain over the phase's groups, in order (A8:59): row = fma(a32, sw * sx, row)
      if (chain) {
        const float4* a4 = reinterpret_cast<const float4*>(A32 + (cm * 16 + cn) * S);
        const float4* x4 = reinterpret_cast<const float4*>(SXT + ((p & 1) * 8 + cm) * S);
        const uint4* sw4 = SWL + (p & 1) * (PG / 8) * 16;
        // groups in blocks of 8: the next block's words are read while this one is chained
        float4 av[2][2], xv[2][2];
        uint4 sv[2];
        auto rd = [&](int g8, int b) {
          sv[b] = sw4[g8 * 16 + cn];
          av[b][0] = a4[2 * g8];
          av[b][1] = a4[2 * g8 + 1];
          xv[b][0] = x4[2 * g8];
          xv[b][1] = x4[2 * g8 + 1];
        };
        auto steps8 = [&](int b) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float4 a = av[b][e >> 2], x = xv[b][e >> 2];
            const int c = e & 3;
            const float ae = c == 0 ? a.x : (c == 1 ? a.y : (c == 2 ? a.z : a.w));
            const float xe = c == 0 ? x.x : (c == 1 ? x.y : (c == 2 ? x.z : x.w));
            acc = fmaf(ae, a8_scale(sv[b], e) * xe, acc);
          }
        };
        if (ng == PG) {
          rd(0, 0);
#pragma unroll
          for (int g8 = 0; g8 < PG / 8; ++g8) {
            if (g8 + 1 < PG / 8) rd(g8 + 1, (g8 + 1) & 1);
            steps8(g8 & 1);
          }
        } else {
          for (int g8 = 0; g8 < ng / 8; ++g8) {  // (ng is a multiple of 8)
            rd(g8, 0);
            steps8(0);
          }
        }
      }
    } else if (p + 1 < nph) {
      quant(p + 1);  // the products of phase p are done with AQL; its scales stay in the other half
    }
    if (p + 2 < nph) {
      issue_x(p + 2);
      issue_s(p + 2);
    }
  }
  if (chain) {
    float* y = j == 0 ? a.y[0] : (j == 1 ? a.y[1] : a.y[2]);
    const int ldy = j == 0 ? a.ldy[0] : (j == 1 ? a.ldy[1] : a.ldy[2]);
    const int n = 16 * mt + cn;
    y[(size_t)cm * ldy + (((a.yperm >> j) & 1) ? head16_index(n) : n)] = acc;
  }
}

// ---- a product with the norm prologue (K = H: one phase of G = 48 groups) ----
// Block: CG a8 tiles of 16 outputs (CG = 4: the gate and up tiles of 32 pairs, column group cg the
// tile cg / 2 of the block's pairs in the gate (cg even) or up (cg odd) matrix: one 512-thread block
// per CU for the 192 blocks of a 6144-wide MLP; CG = 2 for wider ones),
// all M rows, 512 threads.  Wave w multiplies the (column group, chunk) units w + 8k.
// LDS: U (the prologue's rows [8][A8_XPS], then A32 [48][CG][8][16]), AQ [48][A8N_QS] uint64 (word h
// of row m at 8 h + m: a wave's operand reads of one group are 32 consecutive words),
// SXL [48][8], SWL [CG][6][16] uint4, YL [CG][8][16]
constexpr int A8_XPS = 1600;  // row stride of the prologue's rows in LDS (16 RMS chains of 100)
constexpr int A8N_QS = 33;    // operand words per group in LDS (32 + 1: the quantisation stores of
                              // consecutive groups on distinct banks)
template <int CG>
constexpr int a8n_ufloats() {
  return (48 * CG * 8 * 16 > 8 * A8_XPS) ? 48 * CG * 8 * 16 : 8 * A8_XPS;
}
template <int CG>
constexpr size_t a8n_lds() {
  return (size_t)a8n_ufloats<CG>() * 4 + (size_t)48 * A8N_QS * 8 + (size_t)48 * 8 * 4 + (size_t)CG * 6 * 16 * 16 +
         (size_t)CG * 8 * 16 * 4;
}
template <int XM, int CG>
__global__ __launch_bounds__(512) void k_gemv_a8n(GemvTArgs a) {
  constexpr int G = H / 32, GC4 = G / 4, G8 = G / 8, NU = (CG * GC4 + 7) / 8;
  extern __shared__ float4 lds4[];
  float* U = reinterpret_cast<float*>(lds4);
  uint64_t* AQ = reinterpret_cast<uint64_t*>(U + a8n_ufloats<CG>());
  float* SXL = reinterpret_cast<float*>(AQ + G * A8N_QS);
  uint4* SWL = reinterpret_cast<uint4*>(SXL + G * 8);
  float* YL = reinterpret_cast<float*>(SWL + CG * G8 * 16);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int M = a.M;

  // column group cg: matrix mj (pairs: cg % 2) and 16-row tile mt (pairs: the block's first tile
  // plus cg / 2)
  constexpr bool PAIRS = CG >= 2;
  int mj0, mt0;
  {
    const int t = blockIdx.x, tl1 = a.mat[0].N / 16, tl2 = tl1 + a.mat[1].N / 16;
    mj0 = PAIRS ? 0 : (t >= tl1) + (t >= tl2);
    mt0 = PAIRS ? (CG / 2) * t : t - (mj0 == 0 ? 0 : (mj0 == 1 ? tl1 : tl2));
  }
  auto matw = [&](int cg) -> const uint4* {
    const int j = PAIRS ? (cg & 1) : mj0, mt = PAIRS ? mt0 + (cg >> 1) : mt0;
    return (j == 0 ? a.mat[0].w : (j == 1 ? a.mat[1].w : a.mat[2].w)) + (size_t)mt * GC4 * 64 + lane;
  };
  auto mats = [&](int cg) -> const uint4* {
    const int j = PAIRS ? (cg & 1) : mj0, mt = PAIRS ? mt0 + (cg >> 1) : mt0;
    return (j == 0 ? a.mat[0].s : (j == 1 ? a.mat[1].s : a.mat[2].s)) + (size_t)mt * G8 * 16;
  };
  // this wave's units u = w + 8k: column group u % CG, chunk u / CG
  uint4 wA[NU];
  auto issue_w = [&]() {
#pragma unroll
    for (int k = 0; k < NU; ++k) {
      const int u = w + 8 * k;
      if (u < CG * GC4) wA[k] = matw(u % CG)[(size_t)(u / CG) * 64];
    }
  };
  // the tiles' scales: thread f < CG * 96 stages word f % 96 (word k8 of row r) of tile f / 96
  uint4 swr = make_uint4(0, 0, 0, 0);
  if (tid < CG * G8 * 16) swr = mats(tid / (G8 * 16))[tid % (G8 * 16)];

  {
    // E:1358-1361 (mode 1) / E:1375-1378 with E:1390-1404 (mode 2) / E:1375-1377 (mode 3: x1 is
    // the product's input) for row w, as k_gemv_t's norm prologue forms it; the row goes to U in
    // plain order (stride A8_XPS).  Rows past M are not formed (their operand words are zero).
    constexpr int RW4 = H / 4, PER = RW4 / 64;
    const bool live = w < M;
    const int mr = min(w, M - 1);
    const float4* o4 = reinterpret_cast<const float4*>(a.nrm_o) + (size_t)mr * RW4 + lane;
    const float4* x4 = reinterpret_cast<const float4*>(a.nrm_xin) + (size_t)mr * RW4 + lane;
    const float4* w14 = reinterpret_cast<const float4*>(a.nrm_w1) + lane;
    const float4* w24 = reinterpret_cast<const float4*>(a.nrm_w2) + lane;
    float4 ov[PER], xv[PER];
    if (live) {
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        ov[k] = o4[64 * k];
        xv[k] = x4[64 * k];
      }
    }
    issue_w();
    if (live) {
      float* XR = U + (size_t)w * A8_XPS;
      float* CR = XR;  // E:326-345, chains t = e % 16 at 100 t (see k_gemv_t)
      auto rms_row = [&](const float4 (&v)[PER]) -> float {
#pragma unroll
        for (int k = 0; k < PER; ++k) {
          const float f[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const int e = 4 * (lane + 64 * k) + c;
            CR[(e & 15) * 100 + (e >> 4)] = f[c];
          }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        double part = 0;
        if (lane < 16) {
          const float4* ch = reinterpret_cast<const float4*>(CR + lane * 100);
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
        const double b2 = part + shl_d<4>(part);
        const double c2 = b2 + shl_d<8>(b2);
        const double d2 = c2 + shl_d<2>(c2);
        const double e2 = d2 + shl_d<1>(d2);
        const uint64_t u = as_u64(e2);
        const double ss = as_f64(((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), 0) << 32) |
                                 (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, 0));
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        return 1.0f / sqrtf((float)(ss / H) + 1e-6f);
      };
      const int nmode = a.nrm_mode;
      const bool after_mlp = nmode == 2;
      const float scal = a.nrm_scalar;
      float4 w1[PER];
#pragma unroll
      for (int k = 0; k < PER; ++k) w1[k] = w14[64 * k];
      float4 os[PER];
#pragma unroll
      for (int k = 0; k < PER; ++k) os[k] = make_float4(r16(ov[k].x), r16(ov[k].y), r16(ov[k].z), r16(ov[k].w));
      const float r1 = rms_row(os);
      float4 x1[PER];
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        const float4 o = os[k], wv = w1[k], xr = xv[k];
        float4 v = make_float4(r16(xr.x + r16((o.x * r1) * wv.x)), r16(xr.y + r16((o.y * r1) * wv.y)),
                               r16(xr.z + r16((o.z * r1) * wv.z)), r16(xr.w + r16((o.w * r1) * wv.w)));
        if (after_mlp) v = make_float4(r16(v.x * scal), r16(v.y * scal), r16(v.z * scal), r16(v.w * scal));
        x1[k] = v;
        if (blockIdx.x == 0) reinterpret_cast<float4*>(a.nrm_xout)[(size_t)w * RW4 + lane + 64 * k] = v;
      }
      float4 fin[PER];
      if constexpr (XM == 1) {
#pragma unroll
        for (int k = 0; k < PER; ++k) fin[k] = x1[k];
      } else {
        float4 w2[PER];
#pragma unroll
        for (int k = 0; k < PER; ++k) w2[k] = w24[64 * k];
        const float r2 = rms_row(x1);
#pragma unroll
        for (int k = 0; k < PER; ++k) {
          const float4 tv = x1[k], wv = w2[k];
          float4 v = make_float4((tv.x * r2) * wv.x, (tv.y * r2) * wv.y, (tv.z * r2) * wv.z, (tv.w * r2) * wv.w);
          if (!after_mlp) v = make_float4(r16(v.x), r16(v.y), r16(v.z), r16(v.w));
          fin[k] = v;
        }
      }
#pragma unroll
      for (int k = 0; k < PER; ++k) reinterpret_cast<float4*>(XR)[lane + 64 * k] = fin[k];
    }
    if (tid < CG * G8 * 16) SWL[tid] = swr;
    __syncthreads();
  }
  // quantise the rows: thread (m, g), rows >= M zero
  if (tid < 8 * G) {
    const int m = tid / G, g = tid - m * G;
    uint64_t* aq = AQ + (size_t)g * A8N_QS + m;  // word h at aq[8 h]
    if (m < M) {
      const float4* src = reinterpret_cast<const float4*>(U + (size_t)m * A8_XPS + 32 * g);
      float v[32];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float4 f = src[k];
        v[4 * k] = f.x;
        v[4 * k + 1] = f.y;
        v[4 * k + 2] = f.z;
        v[4 * k + 3] = f.w;
      }
      uint64_t q[4];
      SXL[g * 8 + m] = a8_quant_group(v, q);
#pragma unroll
      for (int h = 0; h < 4; ++h) aq[8 * h] = q[h];
    } else {
#pragma unroll
      for (int h = 0; h < 4; ++h) aq[8 * h] = 0;
      SXL[g * 8 + m] = 0.f;
    }
  }
  __syncthreads();
  // the group dots of this wave's units
  {
    const int ar = lane & 15, ah = lane >> 4;
#pragma unroll
    for (int k = 0; k < NU; ++k) {
      const int u = w + 8 * k, cg = u % CG, cl = u / CG;
      if (u < CG * GC4) {  // (uniform per wave)
        const uint4 wv = wA[k];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int g = 4 * cl + i;
          const uint32_t d = i == 0 ? wv.x : (i == 1 ? wv.y : (i == 2 ? wv.z : wv.w));
          const uint64_t A = ar < 8 ? AQ[(size_t)g * A8N_QS + ah * 8 + ar] : 0;
          const i32x4_t D = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)A, a8_wbytes(d), i32x4_t{0, 0, 0, 0}, 0, 0, 0);
          if (ah < 2) {
            float* o = U + ((size_t)(g * CG + cg) * 8 + 4 * ah) * 16 + ar;
            o[0] = (float)D[0];
            o[16] = (float)D[1];
            o[32] = (float)D[2];
            o[48] = (float)D[3];
          }
        }
      }
    }
  }
  __syncthreads();
  // the chains (A8:59): lane (column group, m, n)
  const int ccg = tid >> 7, cm = (tid >> 4) & 7, cn = tid & 15;
  const bool chain = tid < CG * 128 && cm < M;
  float acc = 0.f;
  if (chain) {
    const float* ap = U + ((size_t)ccg * 8 + cm) * 16 + cn;
#pragma unroll
    for (int k8 = 0; k8 < G8; ++k8) {
      const uint4 s4 = SWL[(ccg * G8 + k8) * 16 + cn];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int g = 8 * k8 + e;
        acc = fmaf(ap[(size_t)g * CG * 128], a8_scale(s4, e) * SXL[g * 8 + cm], acc);
      }
    }
  }
  if constexpr (PAIRS) {  // E:292-299 act = rbf8(rbf8(gelu8(rbf8 g)) * rbf8 u), written staged
    if (tid < CG * 128) YL[(ccg * 8 + cm) * 16 + cn] = acc;
    __syncthreads();
    if (tid < CG * 64 && cm < M) {  // pair tile pt = tid / 128: gate group 2 pt, up group 2 pt + 1
      const int pt = tid >> 7;
      const float g = YL[((2 * pt) * 8 + cm) * 16 + cn], u = YL[((2 * pt + 1) * 8 + cm) * 16 + cn];
      const float act = r16(r16(gelu8(r16(g))) * r16(u));
      a.y[0][(size_t)cm * a.ldy[0] + staged_index(16 * (mt0 + pt) + cn)] = act;
      if (CG == 4) U[cm * 32 + 16 * pt + cn] = act;  // (the chains are done with U)
    }
    if constexpr (CG == 4) {
      // the block's 32 outputs are group mt0 / 2 of every row: quantised here for the down
      // product (engine/w4a8_avx2.h:33-41 on the same floats it would quantise)
      if (a.yq) {  // (uniform)
        __syncthreads();
        if (tid < M) {
          float v[32];
#pragma unroll
          for (int k = 0; k < 32; ++k) v[k] = U[tid * 32 + k];
          uint64_t q[4];
          const size_t gq = (size_t)tid * (a.mat[0].N / 32) + (mt0 >> 1);
          a.yqs[gq] = a8_quant_group(v, q);
#pragma unroll
          for (int hw = 0; hw < 4; ++hw) a.yq[gq * 4 + hw] = q[hw];
        }
      }
    }
  } else if (chain) {
    const int n = 16 * mt0 + cn;
    if constexpr (XM == 1) {  // E:421-427 g2 = r16(r16(gelu8(r16 y)) * r16(pli)), staged
      a.y[0][(size_t)cm * a.ldy[0] + staged_index(n)] =
          r16(r16(gelu8(r16(acc))) * r16(a.epi_pli[(size_t)cm * a.epi_pli_ld + n]));
    } else {
      const int j = mj0;
      float* y = j == 0 ? a.y[0] : (j == 1 ? a.y[1] : a.y[2]);
      const int ldy = j == 0 ? a.ldy[0] : (j == 1 ? a.ldy[1] : a.ldy[2]);
      y[(size_t)cm * ldy + (((a.yperm >> j) & 1) ? head16_index(n) : n)] = acc;
    }
  }
}

// mat[j]: a8 tiles (launch_tile_a8) of matrices with N_j % 16 == 0; gateup: mat[0] the gate and
// mat[1] the up matrix (equal N), y[0] the staged activation; yperm as GemvTArgs says (plain
// outputs only).  A product of staged rows (xs)
// quantises them in each block.  Returns the grid of the product (0: refused, nothing launched).
int launch_gemv_a8(const GemvTArgs& a, hipStream_t st) {
  if (a.M < 1 || a.M > 8 || a.K % 256 || a.mrg_po || (a.yperm && (a.gateup || a.epi_pli))) return 0;
  int tiles = 0;
  for (int j = 0; j < 3; ++j) {
    if (a.mat[j].N % 16 || (a.mat[j].N && (!a.mat[j].w || !a.mat[j].s))) return 0;
    tiles += a.mat[j].N / 16;
  }
  const dim3 b(512);
  if (!a.nrm_mode) {
    if (!(a.xq ? a.xqs != nullptr : a.xs != nullptr) || a.gateup || a.epi_pli || a.K > 32 * A8P_PG * A8P_NPM)
      return 0;
    static bool raised_p = false;  // more than 64 KB of LDS (gfx950: up to 160 KB on request)
    if (!raised_p) {
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemv_a8p<A8P_PG, false>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)a8p_lds<A8P_PG>());
      (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&k_gemv_a8p<A8P_PG, true>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)a8p_lds<A8P_PG>());
      raised_p = true;
    }
    if (a.xq)
      hipLaunchKernelGGL((k_gemv_a8p<A8P_PG, true>), dim3(tiles), b, a8p_lds<A8P_PG>(), st, a);
    else
      hipLaunchKernelGGL((k_gemv_a8p<A8P_PG, false>), dim3(tiles), b, a8p_lds<A8P_PG>(), st, a);
    return tiles;
  }
  if (a.K != H) return 0;
  static bool raised = false;  // the norm variants stage more than 64 KB (gfx950: up to 160 KB on request)
  if (!raised) {
    const void* fns[] = {reinterpret_cast<const void*>(&k_gemv_a8n<0, 4>), reinterpret_cast<const void*>(&k_gemv_a8n<0, 2>),
                         reinterpret_cast<const void*>(&k_gemv_a8n<1, 1>),
                         reinterpret_cast<const void*>(&k_gemv_a8n<0, 1>)};
    for (const void* f : fns) (void)hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, 163840);
    raised = true;
  }
  if (a.gateup) {
    if (a.epi_pli || a.mat[0].N != a.mat[1].N || a.mat[2].N) return 0;
    // 4 tiles a block (each block owns one 32-group of every row, quantised here for down)
    if (a8_gateup_quantises(a.mat[0].N)) {
      const int grid = a.mat[0].N / 32;
      hipLaunchKernelGGL((k_gemv_a8n<0, 4>), dim3(grid), b, (a8n_lds<4>()), st, a);
      return grid;
    }
    if (a.yq) return 0;  // (two tiles a block own half a group)
    const int grid = a.mat[0].N / 16;
    hipLaunchKernelGGL((k_gemv_a8n<0, 2>), dim3(grid), b, (a8n_lds<2>()), st, a);
    return grid;
  }
  if (a.epi_pli) {
    if (a.nrm_mode != 3 || a.mat[1].N || a.mat[2].N) return 0;
    hipLaunchKernelGGL((k_gemv_a8n<1, 1>), dim3(tiles), b, (a8n_lds<1>()), st, a);
  } else {
    if (a.nrm_mode == 3) return 0;
    hipLaunchKernelGGL((k_gemv_a8n<0, 1>), dim3(tiles), b, (a8n_lds<1>()), st, a);
  }
  return tiles;
}

}  // namespace g4v
