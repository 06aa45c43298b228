// g4v_w4a8.hip -- W4A8 (int4 weights x per-group int8 activations) for gfx950.
//
// Restates engine/w4a8_avx2.h: quant (A8:30-42) and tile<MT> (A8:46-61), driven over all rows
// as i8_task does (E:303-309).  Per activation row m and 32-group g:
//   sx = amax / 127, inv = sx > 0 ? 1 / sx : 0, q_i = RNE(x_i * inv) (int8), sum = sum_i q_i
//   a32[m][n][g] = sum_i u[n][i] q[m][i] - 8 sum[m][g]               (exact integer)
//   y[m][n] = fma chain over g in order of  row = fma((float)a32, sw[n][g] * sx[m][g], row)
//
// The integer dot runs on the matrix cores: v_mfma_f32_16x16x32_bf16 over one group (K = 32).
// Operands: q as bf16 (|q| <= 127 is exact in bf16) and the weight nibble u as bf16(128 + u)
// (bit pattern 0x4300 | u, no arithmetic to decode); the accumulator input is -136 sum, so
//   D = sum_i q_i (128 + u_i) - 136 sum = sum_i q_i u_i - 8 sum = a32.
// Every product (<= 143 * 128) and every partial sum (< 2^21) is an integer that fp32 holds
// exactly, so D is exact whatever order the unit adds in.  The fp32 chain over groups then
// runs on the VALU in the reference's order, one fma per (row, output, group).
//
// q never saturates: |x_i| <= amax and amax * RN(1 / RN(amax / 127)) < 127.5, so |q_i| <= 127
// and the reference's int16/int8 saturation (A8:40) and its sum of the unsaturated integers
// agree; q is still clamped to [-128, 127] as A8:40 does.
//
// Weights are re-laid once per matrix (k_tile_a8): per tile of 16 output rows and chunk of
// 4 groups, the 64 lanes of a wave hold 16 contiguous bytes each (one coalesced 1 KB load):
// lane (r = lane % 16, h = lane / 16) gets bytes 4h .. 4h+3 of groups 4c .. 4c+3 of row 16t + r,
// i.e. elements 8h .. 8h+7 of each group: the MFMA's B operand for column r, k-slice h.
#include "g4v_internal.h"

namespace g4v {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;

// within each 8-element k-slice the operands hold elements in the order 0,2,4,6,1,3,5,7
// (low nibbles first, then high nibbles), which keeps the weight decode to byte permutes
__host__ __device__ constexpr int a8_slot_elem(int j) { return j < 4 ? 2 * j : 2 * (j - 4) + 1; }

// orig w [N][K/2] (low nibble = even k), s [N][K/32] bf16  ->
// tw [N/16][G/4][64] uint4, ts [N/16][G/8][16] uint4 (8 scales of one row)
__global__ void k_tile_a8(const uint8_t* __restrict__ w, const uint16_t* __restrict__ s, uint4* __restrict__ tw,
                          uint4* __restrict__ ts, int N, int K) {
  const int G = K / 32, GC = G / 4, G8 = G / 8;
  const size_t total = (size_t)(N / 16) * GC * 64;
  for (size_t u = (size_t)blockIdx.x * blockDim.x + threadIdx.x; u < total; u += (size_t)gridDim.x * blockDim.x) {
    const int lane = (int)(u & 63);
    const size_t tc = u >> 6;
    const int c = (int)(tc % GC);
    const size_t t = tc / GC;
    const int r = lane & 15, h = lane >> 4;
    const uint8_t* row = w + (size_t)(t * 16 + r) * (K / 2);
    uint32_t d[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) d[i] = *reinterpret_cast<const uint32_t*>(row + (4 * c + i) * 16 + 4 * h);
    tw[u] = make_uint4(d[0], d[1], d[2], d[3]);
    if (h == 0 && c < G8 * 2 && (c & 1) == 0) {
      const uint4* sr = reinterpret_cast<const uint4*>(s + (size_t)(t * 16 + r) * G);
      ts[(t * G8 + c / 2) * 16 + r] = sr[c / 2];
    }
  }
}

void launch_tile_a8(const uint8_t* w, const uint16_t* s, uint4* tw, uint4* ts, int N, int K, hipStream_t st) {
  const size_t total = (size_t)(N / 16) * (K / 128) * 64;
  int grid = (int)((total + 255) / 256);
  if (grid > 65536) grid = 65536;
  hipLaunchKernelGGL(k_tile_a8, dim3(grid), dim3(256), 0, st, w, s, tw, ts, N, K);
}

// A8:30-42 per (row m, group g); rows M .. Mpad-1 are written as zeros (the MFMA reads them).
// xqb [Mpad][K] bf16 in the slot order; sxt / corr [G][Mpad]; optional q [M][K] int8 (plain
// order), sx / sum [M][G] for the quant entry point.
__global__ void k_w4a8_quant(const float* __restrict__ x, int M, int Mpad, int K, uint16_t* __restrict__ xqb,
                             float* __restrict__ sxt, float* __restrict__ corr, int8_t* __restrict__ qo,
                             float* __restrict__ sxo, int32_t* __restrict__ sumo) {
  const int G = K / 32;
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= Mpad * G) return;
  const int m = idx / G, g = idx - m * G;
  uint4* dst = reinterpret_cast<uint4*>(xqb + (size_t)m * K + 32 * g);
  if (m >= M) {
#pragma unroll
    for (int i = 0; i < 4; ++i) dst[i] = make_uint4(0, 0, 0, 0);
    sxt[(size_t)g * Mpad + m] = 0.f;
    corr[(size_t)g * Mpad + m] = 0.f;
    return;
  }
  const float4* p = reinterpret_cast<const float4*>(x + (size_t)m * K + 32 * g);
  float v[32];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 f = p[i];
    v[4 * i] = f.x;
    v[4 * i + 1] = f.y;
    v[4 * i + 2] = f.z;
    v[4 * i + 3] = f.w;
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
  const float sx = amax / 127.0f, inv = sx > 0.f ? 1.0f / sx : 0.0f;
  int q[32];
  int sum = 0;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    q[i] = (int)__builtin_rintf(v[i] * inv);  // RNE, as _mm256_cvtps_epi32 in the default mode
    sum += q[i];
    q[i] = q[i] > 127 ? 127 : (q[i] < -128 ? -128 : q[i]);
  }
  uint32_t packed[16];
#pragma unroll
  for (int sl = 0; sl < 4; ++sl)
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      const uint32_t b0 = as_u32((float)q[8 * sl + a8_slot_elem(j)]) >> 16;
      const uint32_t b1 = as_u32((float)q[8 * sl + a8_slot_elem(j + 1)]) >> 16;
      packed[sl * 4 + j / 2] = b0 | (b1 << 16);
    }
#pragma unroll
  for (int i = 0; i < 4; ++i) dst[i] = make_uint4(packed[4 * i], packed[4 * i + 1], packed[4 * i + 2], packed[4 * i + 3]);
  sxt[(size_t)g * Mpad + m] = sx;
  corr[(size_t)g * Mpad + m] = (float)(-136 * sum);
  if (qo) {
    uint32_t* qd = reinterpret_cast<uint32_t*>(qo + (size_t)m * K + 32 * g);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      qd[i] = (uint32_t)(q[4 * i] & 0xFF) | ((uint32_t)(q[4 * i + 1] & 0xFF) << 8) |
              ((uint32_t)(q[4 * i + 2] & 0xFF) << 16) | ((uint32_t)(q[4 * i + 3] & 0xFF) << 24);
    sxo[(size_t)m * G + g] = sx;
    sumo[(size_t)m * G + g] = sum;
  }
}

void launch_w4a8_quant(const float* x, int M, int Mpad, int K, uint16_t* xqb, float* sxt, float* corr, int8_t* qo,
                       float* sxo, int32_t* sumo, hipStream_t st) {
  const int n = Mpad * (K / 32);
  hipLaunchKernelGGL(k_w4a8_quant, dim3((n + 127) / 128), dim3(128), 0, st, x, M, Mpad, K, xqb, sxt, corr, qo, sxo,
                     sumo);
}

// bf16(128 + u) for the four low (sel 0x04010400 / 0x04030402 of the lo word) or high nibbles
__device__ __forceinline__ bf16x8_t a8_decode(uint32_t d) {
  const uint32_t lo = d & 0x0F0F0F0Fu, hi = (d >> 4) & 0x0F0F0F0Fu, c = 0x43434343u;
  uint4 o;
  o.x = __builtin_amdgcn_perm(c, lo, 0x04010400u);  // elements 0, 2
  o.y = __builtin_amdgcn_perm(c, lo, 0x04030402u);  // 4, 6
  o.z = __builtin_amdgcn_perm(c, hi, 0x04010400u);  // 1, 3
  o.w = __builtin_amdgcn_perm(c, hi, 0x04030402u);  // 5, 7
  return __builtin_bit_cast(bf16x8_t, o);
}

// One wave per 16 output columns (tile t) and MT m-tiles of 16 rows (rows m0 .. m0 + 16 MT - 1).
// Lane (r, h): B column r, A row r, k-slice h; D element i = row 4h + i, column r.
template <int MT>
__global__ __launch_bounds__(256) void k_w4a8_gemm(const uint4* __restrict__ tw, const uint4* __restrict__ ts,
                                                   const uint16_t* __restrict__ xqb, const float* __restrict__ sxt,
                                                   const float* __restrict__ corr, float* __restrict__ y, int M,
                                                   int Mpad, int N, int K, int ldy) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= N / 16) return;  // whole waves; the kernel has no block-level barrier
  const int m0 = blockIdx.y * 16 * MT;
  const int r = lane & 15, h = lane >> 4;
  const int G = K / 32;
  const uint4* wp = tw + (size_t)t * (G / 4) * 64 + lane;  // chunk c at + 64 c
  const uint4* sp = ts + (size_t)t * (G / 8) * 16 + r;     // scales of groups 8 c8 .. at + 16 c8
  const uint16_t* ap = xqb + (size_t)(m0 + r) * K + 8 * h;  // m-tile mt, group g at + 16 mt K + 32 g
  const int mrow = m0 + 4 * h;                              // + 16 mt: first D row of the lane
  float acc[MT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[mt][i] = 0.f;

  uint4 wv = wp[0], sv = sp[0];
  for (int c = 0; c < G / 4; ++c) {
    const uint4 wcur = wv, scur = sv;
    if (c + 1 < G / 4) wv = wp[(size_t)(c + 1) * 64];
    if ((c & 1) && c + 1 < G / 4) sv = sp[(size_t)((c + 1) >> 1) * 16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int g = 4 * c + i;
      const uint32_t d = i == 0 ? wcur.x : (i == 1 ? wcur.y : (i == 2 ? wcur.z : wcur.w));
      const bf16x8_t B = a8_decode(d);
      const int gi = 4 * (c & 1) + i;  // group within the 8 scales of scur
      const uint32_t s2 = gi < 2 ? scur.x : (gi < 4 ? scur.y : (gi < 6 ? scur.z : scur.w));
      const float sw = as_f32((gi & 1) ? (s2 & 0xFFFF0000u) : (s2 << 16));
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const uint4 av = *reinterpret_cast<const uint4*>(ap + (size_t)mt * 16 * K + 32 * g);
        const float4 cr = *reinterpret_cast<const float4*>(corr + (size_t)g * Mpad + mrow + 16 * mt);
        const float4 sx = *reinterpret_cast<const float4*>(sxt + (size_t)g * Mpad + mrow + 16 * mt);
        const f32x4_t cin = {cr.x, cr.y, cr.z, cr.w};
        const f32x4_t a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av), B, cin, 0, 0, 0);
        acc[mt][0] = fmaf(a[0], sw * sx.x, acc[mt][0]);  // A8:59 sc = sw * sx, row = fma(a32, sc, row)
        acc[mt][1] = fmaf(a[1], sw * sx.y, acc[mt][1]);
        acc[mt][2] = fmaf(a[2], sw * sx.z, acc[mt][2]);
        acc[mt][3] = fmaf(a[3], sw * sx.w, acc[mt][3]);
      }
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = mrow + 16 * mt + i;
      if (m < M) y[(size_t)m * ldy + 16 * t + r] = acc[mt][i];
    }
}

// LDS-staged variant for long M (prefill): a block of 4 waves covers 64 rows (MT = 4 m-tiles)
// and 4 x NT 16-column tiles (NT = 2: 145 VGPRs, 3 waves per SIMD).  The block's activation fragments, corrections and row scales of
// a chunk of 4 groups are loaded once per block (not once per wave) a chunk ahead into
// registers, then written to the other half of a double-buffered LDS stage; one barrier per
// chunk.  Same arithmetic, in the same order, as k_w4a8_gemm.
constexpr int A8_ROWB = 128 * 2 + 16;  // bytes of one staged row: 4 groups x 32 bf16, + pad
template <int NT>
__global__ __launch_bounds__(256) void k_w4a8_gemm_lds(const uint4* __restrict__ tw, const uint4* __restrict__ ts,
                                                       const uint16_t* __restrict__ xqb, const float* __restrict__ sxt,
                                                       const float* __restrict__ corr, float* __restrict__ y, int M,
                                                       int Mpad, int N, int K, int ldy) {
  constexpr int MT = 4;
  __shared__ __align__(16) uint8_t As[2][64 * A8_ROWB];
  __shared__ __align__(16) float Cs[2][4][64], Ss[2][4][64];
  const int lane = threadIdx.x & 63, tid = threadIdx.x;
  const int t0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * NT;  // first 16-column tile of the wave
  const bool active = t0 < N / 16;                            // idle waves still stage and wait
  const int m0 = blockIdx.y * 64;
  const int r = lane & 15, h = lane >> 4;
  const int G = K / 32, NC = G / 4;
  const int tt0 = active ? t0 : 0;
  const uint4* wp = tw + (size_t)tt0 * (G / 4) * 64 + lane;
  const uint4* sp = ts + (size_t)tt0 * (G / 8) * 16 + r;
  // staging roles: thread tid loads 16-byte pieces tid, tid + 256, tid + 512, tid + 768 of the
  // 64 x 256-byte chunk (row = piece / 16, column piece % 16), i.e. column tid % 16 of rows
  // tid / 16 + 16 k, and entry tid of the 4 x 64 corrections / scales
  const int sg = tid >> 6, sm = tid & 63;
  const uint16_t* arow = xqb + (size_t)(m0 + (tid >> 4)) * K + 8 * (tid & 15);  // piece tid; + 16 rows per k
  const int aoff = (tid >> 4) * A8_ROWB + 16 * (tid & 15);
  float acc[MT][NT][4];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int u = 0; u < NT; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[mt][u][i] = 0.f;
  uint4 wv[NT], sv[NT];
#pragma unroll
  for (int u = 0; u < NT; ++u) {
    wv[u] = wp[(size_t)u * (G / 4) * 64];
    sv[u] = sp[(size_t)u * (G / 8) * 16];
  }
  uint4 a0 = *reinterpret_cast<const uint4*>(arow), a1 = *reinterpret_cast<const uint4*>(arow + 16 * K),
        a2 = *reinterpret_cast<const uint4*>(arow + 32 * K), a3 = *reinterpret_cast<const uint4*>(arow + 48 * K);
  float crn = corr[(size_t)sg * Mpad + m0 + sm], sxn = sxt[(size_t)sg * Mpad + m0 + sm];
  *reinterpret_cast<uint4*>(&As[0][aoff]) = a0;
  *reinterpret_cast<uint4*>(&As[0][aoff + 16 * A8_ROWB]) = a1;
  *reinterpret_cast<uint4*>(&As[0][aoff + 32 * A8_ROWB]) = a2;
  *reinterpret_cast<uint4*>(&As[0][aoff + 48 * A8_ROWB]) = a3;
  Cs[0][sg][sm] = crn;
  Ss[0][sg][sm] = sxn;
  __syncthreads();
  for (int c = 0; c < NC; ++c) {
    const int b = c & 1;
    if (c + 1 < NC) {  // uniform: the next chunk's rows, corrections and scales
      const uint16_t* an = arow + 128 * (c + 1);
      a0 = *reinterpret_cast<const uint4*>(an);
      a1 = *reinterpret_cast<const uint4*>(an + 16 * K);
      a2 = *reinterpret_cast<const uint4*>(an + 32 * K);
      a3 = *reinterpret_cast<const uint4*>(an + 48 * K);
      crn = corr[(size_t)(4 * (c + 1) + sg) * Mpad + m0 + sm];
      sxn = sxt[(size_t)(4 * (c + 1) + sg) * Mpad + m0 + sm];
    }
    uint4 wcur[NT], scur[NT];
#pragma unroll
    for (int u = 0; u < NT; ++u) {
      wcur[u] = wv[u];
      scur[u] = sv[u];
      if (c + 1 < NC) wv[u] = wp[((size_t)u * (G / 4) + c + 1) * 64];
      if ((c & 1) && c + 1 < NC) sv[u] = sp[((size_t)u * (G / 8) + ((c + 1) >> 1)) * 16];
    }
    if (active) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int gi = 4 * (c & 1) + i;
        bf16x8_t B[NT];
        float sw[NT];
#pragma unroll
        for (int u = 0; u < NT; ++u) {
          const uint32_t d = i == 0 ? wcur[u].x : (i == 1 ? wcur[u].y : (i == 2 ? wcur[u].z : wcur[u].w));
          B[u] = a8_decode(d);
          const uint32_t s2 = gi < 2 ? scur[u].x : (gi < 4 ? scur[u].y : (gi < 6 ? scur[u].z : scur[u].w));
          sw[u] = as_f32((gi & 1) ? (s2 & 0xFFFF0000u) : (s2 << 16));
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const uint4 av = *reinterpret_cast<const uint4*>(&As[b][(16 * mt + r) * A8_ROWB + 64 * i + 16 * h]);
          const float4 cr = *reinterpret_cast<const float4*>(&Cs[b][i][16 * mt + 4 * h]);
          const float4 sx = *reinterpret_cast<const float4*>(&Ss[b][i][16 * mt + 4 * h]);
          const f32x4_t cin = {cr.x, cr.y, cr.z, cr.w};
          const bf16x8_t A = __builtin_bit_cast(bf16x8_t, av);
#pragma unroll
          for (int u = 0; u < NT; ++u) {
            const f32x4_t a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, B[u], cin, 0, 0, 0);
            acc[mt][u][0] = fmaf(a[0], sw[u] * sx.x, acc[mt][u][0]);  // A8:59
            acc[mt][u][1] = fmaf(a[1], sw[u] * sx.y, acc[mt][u][1]);
            acc[mt][u][2] = fmaf(a[2], sw[u] * sx.z, acc[mt][u][2]);
            acc[mt][u][3] = fmaf(a[3], sw[u] * sx.w, acc[mt][u][3]);
          }
        }
      }
    }
    if (c + 1 < NC) {  // the other half: last read before the previous barrier
      *reinterpret_cast<uint4*>(&As[b ^ 1][aoff]) = a0;
      *reinterpret_cast<uint4*>(&As[b ^ 1][aoff + 16 * A8_ROWB]) = a1;
      *reinterpret_cast<uint4*>(&As[b ^ 1][aoff + 32 * A8_ROWB]) = a2;
      *reinterpret_cast<uint4*>(&As[b ^ 1][aoff + 48 * A8_ROWB]) = a3;
      Cs[b ^ 1][sg][sm] = crn;
      Ss[b ^ 1][sg][sm] = sxn;
    }
    __syncthreads();
  }
  if (!active) return;
  const int mrow = m0 + 4 * h;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int u = 0; u < NT; ++u)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = mrow + 16 * mt + i;
        if (m < M) y[(size_t)m * ldy + 16 * (t0 + u) + r] = acc[mt][u][i];
      }
}

// y [M][ldy] from the quantised rows; Mpad = M rounded up to 16 MT for the chosen MT
// Decode rows (M <= 8, Mpad 16): one block per 16-column tile t.  The tile's K walk is split by
// phases of DEC_PG groups: the sixteen waves compute the phase's group dots (exact integers, the
// same MFMA and operands as k_w4a8_gemm<1>) and the factors sc = sw * sx, and store them for
// rows 0..7 in LDS; after a barrier lane (m, r) of the first 128 threads continues its chain
// row = fma(a32, sc, row) over the phase's groups in group order (A8:59).  Every value and every
// rounding is the one k_w4a8_gemm<1> computes; the group dots of a phase run on sixteen waves at
// once instead of one after another.  K % 256 == 0 (whole chunks of 4 groups, scale blocks of 8).
// Up to three matrices of the same input in one launch (i8_task over nj matrices, E:303-309):
// block b runs tile b - t0[j] of matrix j, t0[j] <= b < t0[j + 1], t0[j + 1] - t0[j] = N_j / 16.
constexpr int DEC_PG = 64;
__global__ __launch_bounds__(1024) void k_w4a8_dec(A8Dec m, const uint16_t* __restrict__ xqb,
                                                  const float* __restrict__ sxt, const float* __restrict__ corr,
                                                  int M, int Mpad, int K) {
  __shared__ float2 S[DEC_PG][32][4];  // [group in phase][lane of rows 0..7][D register]: (a32, sc)
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int b = blockIdx.x;  // gridDim.x == t0[n]
  const int j = b < m.t0[1] ? 0 : (b < m.t0[2] ? 1 : 2);
  const int t = b - m.t0[j];
  const uint4* __restrict__ tw = m.tw[j];
  const uint4* __restrict__ ts = m.ts[j];
  float* __restrict__ y = m.y[j];
  const int ldy = m.ldy[j];
  const int r = lane & 15, h = lane >> 4;
  const int G = K / 32;
  const uint4* wp = tw + (size_t)t * (G / 4) * 64 + lane;  // chunk c at + 64 c
  const uint4* sp = ts + (size_t)t * (G / 8) * 16 + r;     // scales of groups 8 c8 .. at + 16 c8
  const uint16_t* ap = xqb + (size_t)r * K + 8 * h;         // group g at + 32 g
  const int mrow = 4 * h;
  const int cm = tid >> 4, cr = tid & 15;                   // chain lane: row cm, column cr
  const int cl = ((cm >> 2) << 4) | cr, ci = cm & 3;
  float acc = 0.f;
  for (int p = 0; p < G; p += DEC_PG) {
    const int nc = min(DEC_PG, G - p) / 4;  // chunks in this phase
    for (int q = w; q < nc; q += 16) {
      const int c = p / 4 + q;
      const uint4 wcur = wp[(size_t)c * 64];
      const uint4 scur = sp[(size_t)(c >> 1) * 16];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int g = 4 * c + i;
        const uint32_t d = i == 0 ? wcur.x : (i == 1 ? wcur.y : (i == 2 ? wcur.z : wcur.w));
        const bf16x8_t B = a8_decode(d);
        const int gi = 4 * (c & 1) + i;
        const uint32_t s2 = gi < 2 ? scur.x : (gi < 4 ? scur.y : (gi < 6 ? scur.z : scur.w));
        const float sw = as_f32((gi & 1) ? (s2 & 0xFFFF0000u) : (s2 << 16));
        const uint4 av = *reinterpret_cast<const uint4*>(ap + 32 * (size_t)g);
        const float4 crv = *reinterpret_cast<const float4*>(corr + (size_t)g * Mpad + mrow);
        const float4 sx = *reinterpret_cast<const float4*>(sxt + (size_t)g * Mpad + mrow);
        const f32x4_t cin = {crv.x, crv.y, crv.z, crv.w};
        const f32x4_t a = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av), B, cin, 0, 0, 0);
        if (h < 2) {
          float2* o = S[g - p][lane];
          o[0] = make_float2(a[0], sw * sx.x);
          o[1] = make_float2(a[1], sw * sx.y);
          o[2] = make_float2(a[2], sw * sx.z);
          o[3] = make_float2(a[3], sw * sx.w);
        }
      }
    }
    __syncthreads();
    if (tid < 128) {
      const int ng = nc * 4;
#pragma unroll 8
      for (int gi = 0; gi < ng; ++gi) {
        const float2 v = S[gi][cl][ci];
        acc = fmaf(v.x, v.y, acc);
      }
    }
    __syncthreads();
  }
  if (tid < 128 && cm < M) y[(size_t)cm * ldy + 16 * t + cr] = acc;
}

int w4a8_mt(int M) { return M <= 16 ? 1 : (M <= 64 ? 2 : 4); }
int w4a8_mpad(int M) {
  const int bm = 16 * w4a8_mt(M);
  return (M + bm - 1) / bm * bm;
}

void launch_w4a8_gemm(const uint4* tw, const uint4* ts, const uint16_t* xqb, const float* sxt, const float* corr,
                      float* y, int M, int N, int K, int ldy, hipStream_t st) {
  const int MT = w4a8_mt(M), Mpad = w4a8_mpad(M);
  if (M <= 8 && N % 16 == 0 && K % 256 == 0) {  // decode rows: group dots split over the block's waves
    A8Dec m{};
    m.tw[0] = tw;
    m.ts[0] = ts;
    m.y[0] = y;
    m.ldy[0] = ldy;
    m.t0[1] = m.t0[2] = m.t0[3] = N / 16;
    hipLaunchKernelGGL(k_w4a8_dec, dim3(N / 16), dim3(1024), 0, st, m, xqb, sxt, corr, M, Mpad, K);
    return;
  }
  if (MT == 4 && (N / 16) % 2 == 0 && K % 128 == 0) {  // long M: 4 x 2 tiles per wave, staged rows
    const dim3 grid((N / 16 / 2 + 3) / 4, Mpad / 64);
    hipLaunchKernelGGL(k_w4a8_gemm_lds<2>, grid, dim3(256), 0, st, tw, ts, xqb, sxt, corr, y, M, Mpad, N, K, ldy);
    return;
  }
  const dim3 grid((N / 16 + 3) / 4, Mpad / (16 * MT));
  switch (MT) {
    case 1:
      hipLaunchKernelGGL(k_w4a8_gemm<1>, grid, dim3(256), 0, st, tw, ts, xqb, sxt, corr, y, M, Mpad, N, K, ldy);
      break;
    case 2:
      hipLaunchKernelGGL(k_w4a8_gemm<2>, grid, dim3(256), 0, st, tw, ts, xqb, sxt, corr, y, M, Mpad, N, K, ldy);
      break;
    default:
      hipLaunchKernelGGL(k_w4a8_gemm<4>, grid, dim3(256), 0, st, tw, ts, xqb, sxt, corr, y, M, Mpad, N, K, ldy);
      break;
  }
}

int launch_w4a8_dec(const A8Dec& m, int n, const uint16_t* xqb, const float* sxt, const float* corr, int M, int K,
                    hipStream_t st) {
  if (n < 1 || n > 3 || M < 1 || M > 8 || K % 256) return 0;
  hipLaunchKernelGGL(k_w4a8_dec, dim3(m.t0[n]), dim3(1024), 0, st, m, xqb, sxt, corr, M, w4a8_mpad(M), K);
  return 1;
}

}  // namespace g4v
