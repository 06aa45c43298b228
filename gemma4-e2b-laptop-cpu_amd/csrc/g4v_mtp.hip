// g4v_mtp.hip -- the MTP drafter step (draft_step, E:1534-1563) on gfx950.
//
// One draft step on the device, so that a chain of drafts runs without host round trips:
//   comb = [r16(E[tok] * sqrt(1536)), h]  ->  dx = r16(pre . comb)                   (E:1537-1539)
//   4 layers: da = rms(dx, in_ln); q = q_proj . da; per head r16-norm + RoPE at pos;
//     attention over the target's KV cache (layer 13, the global drafter layer: 14), split-KV
//     with T splits, keys [lo, P]; o = r16(o_proj . att); dx = r16(dx + r16(rms(o, post_attn)));
//     da = r16(rms(dx, pre_ff)); act = r16(r16(gelu8(r16 gate)) * r16 up); o = r16(down . act);
//     dx = r16(dx + r16(rms(o, post_ff))); dx = r16(dx * scalar)                    (E:1540-1550)
//   dh = r16(rms(dx, norm)); b_out = r16(post . dh); centroid scores = cent . dh  (E:1551-1553)
//   top-32 centroids (descending score, earlier index first), their 32 x 128 tokens scored
//   against dh, the first maximum is the draft; the runner-up follows the engine's scan
//   (E:1554-1559).
// Every bf16 product is b16_rows (E:586-614): per output, two 8-lane FMA chains over k in steps
// of 16 (k = 16 s + l and 16 s + 8 + l), summed lane-wise, then hsum.  Here 16 lanes of a wave
// hold the 16 chains of one output, so a 256-thread block computes 16 outputs.
#include "g4v_layer.h"

namespace g4v {

namespace {

// input prologue: x; rms(x, nw); r16(rms(x, nw)); [r16(E[*tok] sqrt H), x]; and the residual
// blocks of a drafter layer folded in front of the next product (K = 256, x = dx):
//   RES0 (E:1545-1546): v = r16(x + r16(rms(r16(yin), w1))); input r16(rms(v, nw))
//   RES1 (E:1548-1550): v = r16(r16(x + r16(rms(r16(yin), w1))) * scalar); input rms(v, nw)
//   RES1_R16: as RES1, input r16(rms(v, nw))
// block 0 stores v to dxout (a different buffer from x: other blocks still read x)
enum { B16_PLAIN = 0, B16_RMS = 1, B16_RMS_R16 = 2, B16_COMB = 3, B16_RES0 = 4, B16_RES1 = 5, B16_RES1_R16 = 6 };
enum { B16_STORE = 0, B16_R16 = 1, B16_GATEUP = 2 };                  // output epilogue

struct B16Args {
  const uint16_t* W;   // [rows][K] bf16
  const uint16_t* W2;  // B16_GATEUP: the up matrix
  const int* rows;     // row of output n, or null: row n (or, with top: order[top[n / 128] 128 + n % 128])
  const int* top;
  const int* order;
  int N, K;
  const float* x;      // input [K], or the prologue's source
  const float* nw;     // norm weights (B16_RMS*)
  const uint16_t* E;   // B16_COMB: token embedding [V][1536] ...
  const int* tok;      // ... of token *tok, followed by x [1536]
  float* y;
  float* xout;         // optional: block 0 stores the staged input
  const float* yin;    // RES*: the previous product's output [256]
  const float* w1;     // RES*: post_attn / post_ff
  float* dxout;        // RES*: the updated residual (block 0)
  float scalar;        // RES1*: the layer scalar
};

constexpr int B16_MAXK = 3072;
constexpr int DR_MAXC = 4096;  // centroids

template <int PRO, int EPI>
__global__ __launch_bounds__(256) void k_b16(B16Args a) {
  __shared__ __align__(16) float xs[B16_MAXK];
  __shared__ double red[16];
  const int K = a.K;
  if (PRO == B16_COMB) {
    const int tk = *a.tok;
    const float sqh = sqrtf((float)H);
    for (int i = threadIdx.x; i < H; i += 256) {
      xs[i] = r16(bf2f(a.E[(size_t)tk * H + i]) * sqh);  // E:1537
      xs[H + i] = a.x[i];
    }
  } else if (PRO >= B16_RES0) {  // K == 256 == blockDim.x: thread i owns element i
    const int i = threadIdx.x;
    xs[i] = r16(a.yin[i]);
    __syncthreads();
    const float r1 = rms_inv(block_sumsq(xs, 256, red), 256);
    float v = r16(a.x[i] + r16((xs[i] * r1) * a.w1[i]));
    if (PRO != B16_RES0) v = r16(v * a.scalar);
    if (a.dxout && blockIdx.x == 0) a.dxout[i] = v;
    __syncthreads();  // every thread has read xs
    xs[i] = v;
  } else {
    for (int i = threadIdx.x; i < K; i += 256) xs[i] = a.x[i];
  }
  __syncthreads();
  if (PRO == B16_RMS || PRO == B16_RMS_R16 || PRO >= B16_RES0) {  // E:345: (x * r) * w
    const bool rnd = PRO == B16_RMS_R16 || PRO == B16_RES0 || PRO == B16_RES1_R16;
    const float r = rms_inv(block_sumsq(xs, K, red), K);
    for (int i = threadIdx.x; i < K; i += 256) {
      const float v = (xs[i] * r) * a.nw[i];
      xs[i] = rnd ? r16(v) : v;
    }
    __syncthreads();
  }
  if (a.xout && blockIdx.x == 0)
    for (int i = threadIdx.x; i < K; i += 256) a.xout[i] = xs[i];
  const int n = blockIdx.x * 16 + (threadIdx.x >> 4), l = threadIdx.x & 15;
  const bool live = n < a.N;
  const size_t row = !live ? 0
                     : a.rows ? (size_t)a.rows[n]
                     : a.top  ? (size_t)a.order[(size_t)a.top[n >> 7] * 128 + (n & 127)]
                              : (size_t)n;
  const uint16_t* w = a.W + row * K + l;
  const uint16_t* w2 = EPI == B16_GATEUP ? a.W2 + row * K + l : nullptr;
  float acc = 0.f, acc2 = 0.f;
  if (live) {
    // chain l: elements l, 16 + l, ... in order; the weights of 32 steps are loaded ahead of
    // their FMAs (K is a multiple of 512 here or the tail loop takes the rest)
    int k = 0;
    for (; k + 512 <= K; k += 512) {
      uint16_t wb[32], wb2[32];
#pragma unroll
      for (int u = 0; u < 32; ++u) {
        wb[u] = w[k + 16 * u];
        if (EPI == B16_GATEUP) wb2[u] = w2[k + 16 * u];
      }
#pragma unroll
      for (int u = 0; u < 32; ++u) {
        acc = fmaf(bf2f(wb[u]), xs[k + 16 * u + l], acc);
        if (EPI == B16_GATEUP) acc2 = fmaf(bf2f(wb2[u]), xs[k + 16 * u + l], acc2);
      }
    }
#pragma unroll 8
    for (; k < K; k += 16) {
      acc = fmaf(bf2f(w[k]), xs[k + l], acc);
      if (EPI == B16_GATEUP) acc2 = fmaf(bf2f(w2[k]), xs[k + l], acc2);
    }
  }
  // lanes 0..7 of each 16-lane group: v_l = a_l + b_l, then ((v0+v4)+(v1+v5))+((v2+v6)+(v3+v7))
  auto hsum16 = [](float v) {
    v = v + __shfl_down(v, 8, 16);
    v = v + __shfl_down(v, 4, 16);
    v = v + __shfl_down(v, 1, 16);
    return v + __shfl_down(v, 2, 16);
  };
  const float s = hsum16(acc);
  const float s2 = EPI == B16_GATEUP ? hsum16(acc2) : 0.f;
  if (live && l == 0) {
    if (EPI == B16_STORE) a.y[n] = s;
    else if (EPI == B16_R16) a.y[n] = r16(s);
    else a.y[n] = r16(r16(gelu8(r16(s))) * r16(s2));  // E:669-672
  }
}

// per head (4): x = r16((x * r) * qn), then NeoX RoPE at the step's position (E:1542): P + 1 + j,
// or P + 1 for every step with ENGINE_DRAFT_SAMEPOS (Pp[2] set, E:1516, 1633); D the layer's head
// dim (256, or 512 for the global layer of a drafter checkpoint)
template <int D>
__global__ __launch_bounds__(D) void k_dr_qnorm(float* __restrict__ q, const float* __restrict__ qn,
                                                const float* __restrict__ cs, const float* __restrict__ sn,
                                                const int* __restrict__ Pp, int j) {
  constexpr int NV = 4;
  const int pos = Pp[0] + 1 + (Pp[2] ? 0 : j);
  __shared__ float xv[NV][D];
  __shared__ double part[NV][16];
  __shared__ float rinv[NV];
  const int e = threadIdx.x;
#pragma unroll
  for (int h = 0; h < NV; ++h) xv[h][e] = q[h * D + e];
  __syncthreads();
  if (e < NV * 16) {  // ss_avx2 order (E:326-343): lane t16 sums x[16 i + t16]^2 over i
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
    for (int k = 0; k < 4; ++k) a[k] = (p[k] + p[4 + k]) + (p[8 + k] + p[12 + k]);
    rinv[e] = rms_inv((a[0] + a[2]) + (a[1] + a[3]), D);
  }
  __syncthreads();
  float y[NV];
#pragma unroll
  for (int h = 0; h < NV; ++h) y[h] = r16((xv[h][e] * rinv[h]) * qn[e]);
  __syncthreads();
#pragma unroll
  for (int h = 0; h < NV; ++h) xv[h][e] = y[h];
  __syncthreads();
  const int i2 = e & (D / 2 - 1);
  const float c = cs[(size_t)pos * (D / 2) + i2], sv = sn[(size_t)pos * (D / 2) + i2];
#pragma unroll
  for (int h = 0; h < NV; ++h)
    q[h * D + e] = e < D / 2 ? fmaf(xv[h][e], c, -(xv[h][e + D / 2] * sv)) : fmaf(xv[h][e], c, xv[h][e - D / 2] * sv);
}

// a chain's inputs (E:1631-1633): the hidden state, the first token and, per step j, the
// attention geometry (M = 1, keys [lo, P], lo = pos - 511 clamped at 0 on sliding layers,
// pos = P + 1 + j, E:1543, or P + 1 with ENGINE_DRAFT_SAMEPOS: in[3] set, E:1633)
__global__ __launch_bounds__(256) void k_dr_setup(const int* __restrict__ in, const float* __restrict__ hbase,
                                                  float* __restrict__ hin, int* __restrict__ tok,
                                                  AttnGeom* __restrict__ geo, int k, int T) {
  const int t0 = in[0], P = in[1], hrow = in[2], same = in[3];
  const float* src = hrow >= 0 ? hbase + (size_t)hrow * H : reinterpret_cast<const float*>(in + 4);
  for (int i = threadIdx.x; i < H; i += 256) hin[i] = src[i];
  if (threadIdx.x == 0) tok[0] = t0;
  if (threadIdx.x < 2 * k) {
    const int j = threadIdx.x >> 1, sl = (threadIdx.x & 1) == 0;
    AttnGeom g{};
    g.M = 1;
    g.T = T;
    g.pos[0] = P;
    g.lo[0] = sl ? max(0, P + 1 + (same ? 0 : j) - 511) : 0;
    g.skip_lo[0] = 1;
    g.skip_hi[0] = 0;
    g.kmin = g.lo[0];
    g.kmax = P;
    geo[threadIdx.x] = g;
  }
}

// E:1554-1555 top-32 centroids (descending, equal scores in index order): centroid c's place is
// the count of scores above it plus the equal scores before it.  A block ranks 64 centroids;
// its 4 waves count over the four quarters of the scores (LDS, 4 scores per read).
__global__ __launch_bounds__(256) void k_dr_rank(const float* __restrict__ score, int C, int* __restrict__ top) {
  __shared__ __align__(16) float s[DR_MAXC];
  __shared__ int part[4][64];
  for (int j = threadIdx.x; j < C; j += 256) s[j] = score[j];
  __syncthreads();
  const int cl = threadIdx.x & 63, q = threadIdx.x >> 6, c = blockIdx.x * 64 + cl;
  const float v = c < C ? s[c] : 0.f;
  const int j0 = q * (C / 4), j1 = q == 3 ? C : j0 + C / 4;  // C % 4 == 0
  int rank = 0;
  for (int j = j0; j < j1; j += 4) {
    const float4 u = *reinterpret_cast<const float4*>(&s[j]);
    rank += (u.x > v) || (u.x == v && j < c);
    rank += (u.y > v) || (u.y == v && j + 1 < c);
    rank += (u.z > v) || (u.z == v && j + 2 < c);
    rank += (u.w > v) || (u.w == v && j + 3 < c);
  }
  part[q][cl] = rank;
  __syncthreads();
  if (q == 0 && c < C) {
    rank = (part[0][cl] + part[1][cl]) + (part[2][cl] + part[3][cl]);
    if (rank < 32) top[rank] = c;
  }
}

// E:1557-1559: the first maximum of the candidate scores is the draft.  The engine's scan keeps
// a runner-up: at the maximum's first index i* it becomes the best before i* (or cand[0] at
// -1e30 when i* = 0), then any later score above it replaces it.  So the runner-up is the first
// maximum after i* if that beats the best before i*, else the best before i*.
__global__ __launch_bounds__(1024) void k_dr_best(const float* __restrict__ cs, const int* __restrict__ top,
                                                  const int* __restrict__ order, int nc, int* __restrict__ tok,
                                                  int* __restrict__ sec, float* __restrict__ gap) {
  auto cand = [&](int i) { return order[(size_t)top[i >> 7] * 128 + (i & 127)]; };  // E:1556
  __shared__ float rv[32];
  __shared__ int ri[32];
  auto argmax = [&](int lo, int hi, float& bv, int& bi) {  // first index of the maximum of [lo, hi)
    float v = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = lo + (int)threadIdx.x; i < hi; i += 1024) {
      const float u = cs[i];
      if (u > v) {  // ascending i per thread: keeps the first
        v = u;
        idx = i;
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float v2 = __shfl_xor(v, o);
      const int i2 = __shfl_xor(idx, o);
      if (v2 > v || (v2 == v && i2 < idx)) {
        v = v2;
        idx = i2;
      }
    }
    __syncthreads();
    if ((threadIdx.x & 63) == 0) {
      rv[threadIdx.x >> 6] = v;
      ri[threadIdx.x >> 6] = idx;
    }
    __syncthreads();
    v = rv[0];
    idx = ri[0];
    for (int w = 1; w < 16; ++w)
      if (rv[w] > v || (rv[w] == v && ri[w] < idx)) {
        v = rv[w];
        idx = ri[w];
      }
    bv = v;
    bi = idx;
  };
  float M, M1 = -1e30f, M2 = -INFINITY;
  int is, i1 = 0, i2 = -1;
  argmax(0, nc, M, is);
  if (is > 0) argmax(0, is, M1, i1);
  if (is + 1 < nc) argmax(is + 1, nc, M2, i2);
  if (threadIdx.x == 0) {
    const bool later = i2 >= 0 && M2 > M1;
    *tok = cand(is);
    *sec = later ? cand(i2) : cand(i1);
    *gap = M - (later ? M2 : M1);
  }
}

}  // namespace

void launch_b16(const B16Launch& L, hipStream_t st) {
  B16Args a{L.W, L.W2, L.rows, L.top, L.order, L.N, L.K, L.x, L.nw, L.E, L.tok, L.y, L.xout, L.yin, L.w1, L.dxout,
            L.scalar};
  const dim3 grid((L.N + 15) / 16), block(256);
#define G4V_B16(P, E) hipLaunchKernelGGL((k_b16<P, E>), grid, block, 0, st, a)
  switch (L.pro * 3 + L.epi) {
    case B16_PLAIN * 3 + B16_STORE: G4V_B16(B16_PLAIN, B16_STORE); break;
    case B16_PLAIN * 3 + B16_R16: G4V_B16(B16_PLAIN, B16_R16); break;
    case B16_RMS * 3 + B16_STORE: G4V_B16(B16_RMS, B16_STORE); break;
    case B16_COMB * 3 + B16_R16: G4V_B16(B16_COMB, B16_R16); break;
    case B16_RES0 * 3 + B16_GATEUP: G4V_B16(B16_RES0, B16_GATEUP); break;
    case B16_RES1 * 3 + B16_STORE: G4V_B16(B16_RES1, B16_STORE); break;
    case B16_RES1_R16 * 3 + B16_STORE: G4V_B16(B16_RES1_R16, B16_STORE); break;
    case B16_RES1_R16 * 3 + B16_R16: G4V_B16(B16_RES1_R16, B16_R16); break;
    default: break;  // not used by the drafter
  }
#undef G4V_B16
}

void launch_dr_qnorm(float* q, const float* qn, const float* cs, const float* sn, const int* Pp, int j, int hd,
                     hipStream_t st) {
  if (hd == 512) hipLaunchKernelGGL(k_dr_qnorm<512>, dim3(1), dim3(512), 0, st, q, qn, cs, sn, Pp, j);
  else hipLaunchKernelGGL(k_dr_qnorm<HD>, dim3(1), dim3(HD), 0, st, q, qn, cs, sn, Pp, j);
}
void launch_dr_setup(const int* in, const float* hbase, float* hin, int* tok, AttnGeom* geo, int k, int T,
                     hipStream_t st) {
  hipLaunchKernelGGL(k_dr_setup, dim3(1), dim3(256), 0, st, in, hbase, hin, tok, geo, k, T);
}
void launch_dr_rank(const float* score, int C, int* top, hipStream_t st) {
  hipLaunchKernelGGL(k_dr_rank, dim3((C + 63) / 64), dim3(256), 0, st, score, C, top);
}
void launch_dr_best(const float* cs, const int* top, const int* order, int nc, int* tok, int* sec, float* gap,
                    hipStream_t st) {
  hipLaunchKernelGGL(k_dr_best, dim3(1), dim3(1024), 0, st, cs, top, order, nc, tok, sec, gap);
}

}  // namespace g4v
