// g4v_attn.hip -- split-KV attention over the draft rows (E:743-877) and the exact
// log-sum-exp merge of the splits (E:1019-1059), gfx950.  E = engine/gemma4_engine.cpp.
//
// Split t covers keys [kmin + t*len/T, kmin + (t+1)*len/T) exactly as the reference's
// worker t does, and every per-(row, head) value is produced in the reference's fp32 order:
//   score_p = hsum8(s0 + s1), s0/s1 two 8-lane FMA chains over the head dim in steps of 16;
//   w_p = exp8(score_p - max), l = sum of w_p in position order, o_i = fma chain over p;
//   merge: sc_t = libm expf(max_t - M0), l = sum_t (double) l_t sc_t,
//          out = r16((fma chain over splits of o_t sc_t) * (float)(1 / l)).
// Two kernels: k_attn_rows, the verify pass's attention (q/k norm, RoPE and the pass's cache rows
// fused, partials merged by the o projection), and k_attn_split + k_attn_merge, the split-KV
// attention of the standalone entry points on a geometry given by the caller.  Both visit a
// split's value cache in whole blocks of 32 positions, fetched into registers ahead of use.
#include "g4v_layer.h"

namespace g4v {

__constant__ uint64_t c_expf_tab[32] = G4V_EXPF_TABLE;

constexpr int ATT_THREADS = 256;
constexpr int ATT_TILE = 32;  // positions per tile = one block of the value cache
constexpr int ATT_HB = 2;     // heads per block (224 blocks for a 7-row pass: every CU busy)
constexpr int ATT_PMAX = 2080;  // positions per split held in LDS (6 splits cover 12,480 keys)
constexpr int ATT_SW = ATT_PMAX + 2 * ATT_TILE;  // weight row: a split widened to whole tiles
constexpr int ATT_RING = 4;  // tiles in flight: the split's key tiles, then its value tiles

struct AttnPtrs {
  const uint16_t* KC;  // the layer's cache in the device layout (kc_index / vc_index)
  const uint16_t* VC;
  const float* q;
  int ldq;
  float* po;  // [T][M][NQ][HD]
  float* pm;  // [T][M][NQ]
  float* pl;  // [T][M][NQ]
  float* out; // [M][ldo]
  int ldo;
  float* gs;  // not null: out is written in the staged GEMV input layout, group sums here [M][ldo/32]
  // verify pass (fused E:1307-1324): q, k, v straight from the projection, normalised and
  // rotated here; the pass's own key/value rows are formed in LDS and written to the cache
  const float* kraw;  // [M][HD]
  const float* vraw;  // [M][HD]
  const float* ropestep;  // the step's RoPE factors of the layer type: [MAXM][cos | sin][HD/2]
  const float* qn;    // q_norm / k_norm weights [HD] (the verify pass: in the 16-lane head order)
  const float* kn;
  uint16_t* KCw;      // the layer's cache (same as KC / VC), written for the pass's rows
  uint16_t* VCw;
  const AttnGeom* gdev;  // raw attention: the geometry in device memory (replaces the argument)
  // with gs: the merged rows also quantised for a W4A8 product (engine/w4a8_avx2.h:33-41), the
  // four operand words of group g of row m at xq[(m * ldo / 32 + g) * 4], its scale at xqs
  uint64_t* xq;
  float* xqs;
};

// grid (T, M, NQ / ATT_HB); the geometry as the argument gin or in device memory (P.gdev)
__global__ __launch_bounds__(ATT_THREADS) void k_attn_split(AttnPtrs P, AttnGeom gin, int T) {
  __shared__ float qs[ATT_HB][8][32];              // lane l's 32 query values: s0 chain then s1 chain
  __shared__ __align__(16) float sw[ATT_HB][ATT_SW];
  __shared__ float wmax[ATT_THREADS / 64][ATT_HB];
  __shared__ float smax[ATT_HB];
  const int t = blockIdx.x, m = blockIdx.y, h0 = blockIdx.z * ATT_HB;
  const int e = threadIdx.x;  // element e: chain s = (e/8)%2, step tt = e/16, lane e%8
  // the query heads first, together with the geometry (one round trip)
  float qv[ATT_HB];
#pragma unroll
  for (int hh = 0; hh < ATT_HB; ++hh) qv[hh] = P.q[(size_t)m * P.ldq + (h0 + hh) * HD + e];
  const AttnGeom& G = P.gdev ? *P.gdev : gin;
  const int M = G.M, kmin = G.kmin, kmax = G.kmax, pos_m = G.pos[m], lo_m = G.lo[m], sl_m = G.skip_lo[m],
            sh_m = G.skip_hi[m];
  if (m >= M) return;
  const int len = kmax - kmin + 1;
  // (t + 1) len < 2^31 for every launch: 32-bit division
  const int c0 = kmin + (int)((unsigned)(t * len) / (unsigned)T),
            c1 = kmin + (int)((unsigned)((t + 1) * len) / (unsigned)T);
  const int PP = c1 - c0;
  // E:740 attn_allowed for this block's row, restricted to the split
  auto allowed = [=](int p) { return p >= c0 && p < c1 && p >= lo_m && p <= pos_m && !(p >= sl_m && p <= sh_m); };
  // bit e: position pb + e is inside the split and allowed, for a tile of 32 positions
  auto bits_in = [](int a, int b, int pb) -> uint32_t {  // positions [a, b] within [pb, pb + 31]
    const int lo = max(a - pb, 0), hi = min(b - pb, 31);
    if (lo > hi) return 0u;
    const uint32_t up = hi == 31 ? 0xFFFFFFFFu : ((1u << (hi + 1)) - 1u);
    return up & ~((1u << lo) - 1u);
  };
  auto tile_mask = [=](int pb) -> uint32_t {
    return bits_in(max(lo_m, c0), min(pos_m, c1 - 1), pb) & ~bits_in(sl_m, sh_m, pb);
  };
  // The split is visited in whole blocks of the value cache: tile s covers positions
  // [pb0 + 32 s, pb0 + 32 s + 32); positions outside [c0, c1) are masked.  Two streams of
  // tile loads, ATT_RING tiles each in flight from the start: key tile s in slot s % ATT_RING
  // of the key ring, value tile v in slot v % ATT_RING of the value ring (a split of up to
  // ATT_RING tiles, every sliding-window split, has all of its tiles in flight at once).
  const int pb0 = c0 & ~(ATT_TILE - 1);
  const int NT = PP > 0 ? ((c1 - 1) >> 5) - (c0 >> 5) + 1 : 0;
  const int NTp = (NT + ATT_RING - 1) / ATT_RING * ATT_RING;
  const int ps = threadIdx.x >> 3, l = threadIdx.x & 7;  // key sweep: position ps, chain lane l
  // key tile: lane (ps, l) takes the 64 bytes of chain lane l at position pb + ps (clamped into
  // the split); value tile: lane i takes dim i of the block's 32 positions (4 parts of 16 bytes)
  // Every stream entry issues its four loads, so each ring slot has exactly one definition
  // per tile (no merges that would make the compiler wait on loads still in flight): empty
  // entries and entries past the stream load a row they never use.
  uint4 kring[ATT_RING][4], vring[ATT_RING][4];
  const uint16_t* kbase = P.KC + l * 32;
  const uint16_t* vbase = P.VC + threadIdx.x * 8;
  auto issue_k = [&](int s, uint4 (&r)[4]) {  // entries past the split reload its last row
    const size_t koff = (size_t)max(min(pb0 + min(s, NT - 1) * ATT_TILE + ps, c1 - 1), 0) * HD;
    const uint4* src = reinterpret_cast<const uint4*>(kbase + koff);
#pragma unroll
    for (int c = 0; c < 4; ++c) r[c] = src[c];
  };
  auto issue_v = [&](int v, uint4 (&r)[4]) {  // entries past the split reload its last block
    const size_t voff = (size_t)((pb0 >> 5) + max(min(v, NT - 1), 0)) * (ATT_TILE * HD);
    const uint4* src = reinterpret_cast<const uint4*>(vbase + voff);
#pragma unroll
    for (int c = 0; c < 4; ++c) r[c] = src[c * (8 * HD / 8)];  // part c: 8 HD bf16 further
  };
#pragma unroll
  for (int k = 0; k < ATT_RING; ++k) issue_k(k, kring[k]);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int k = 0; k < ATT_RING; ++k) issue_v(k, vring[k]);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int hh = 0; hh < ATT_HB; ++hh) qs[hh][e & 7][((e >> 3) & 1) * 16 + (e >> 4)] = qv[hh];
  float mymax[ATT_HB];
#pragma unroll
  for (int hh = 0; hh < ATT_HB; ++hh) mymax[hh] = -1e30f;
  __syncthreads();
  float qr[ATT_HB][32];  // this lane's query values of the block's heads
#pragma unroll
  for (int hh = 0; hh < ATT_HB; ++hh)
#pragma unroll
    for (int i = 0; i < 32; ++i) qr[hh][i] = qs[hh][l][i];

  // sweep 1: scores (E:750-816) straight from the fetched key rows; key ring slot k holds
  // key tile s = base + k.  Lane group ps scores position pb + ps (positions outside the split
  // from a clamped row: their scores are never used); its lane 0 keeps the running max over
  // the allowed positions (max is order free).
  for (int base = 0; base < NTp; base += ATT_RING)
#pragma unroll
  for (int k = 0; k < ATT_RING; ++k) {
    const int s = base + k;
    const int pb = pb0 + s * ATT_TILE, p = pb + ps;
    if (s < NT) {  // uniform; otherwise an empty entry
      uint4 kr[4] = {kring[k][0], kring[k][1], kring[k][2], kring[k][3]};
      float kf[32];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint32_t w4[4] = {kr[c].x, kr[c].y, kr[c].z, kr[c].w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          kf[c * 8 + 2 * q] = as_f32(w4[q] << 16);
          kf[c * 8 + 2 * q + 1] = as_f32(w4[q] & 0xFFFF0000u);
        }
      }
#pragma unroll
      for (int hh = 0; hh < ATT_HB; ++hh) {
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int tt = 0; tt < 16; ++tt) {
          s0 = fmaf(qr[hh][tt], kf[tt], s0);
          s1 = fmaf(qr[hh][16 + tt], kf[16 + tt], s1);
        }
        const float v = hsum8_lanes(s0 + s1);
        if (l == 0) {
          sw[hh][p - pb0] = v;
          if (allowed(p) && mymax[hh] < v) mymax[hh] = v;
        }
      }
    }
    // the slot's next entry, once its current one is consumed (the loop then carries each
    // slot in one register set: no copies, which would wait for loads in flight)
    issue_k(s + ATT_RING, kring[k]);
  }
#pragma unroll
  for (int hh = 0; hh < ATT_HB; ++hh) {
    float v = mymax[hh];
    for (int s = 1; s < 64; s <<= 1) v = fmaxf(v, __shfl_xor(v, s, 64));
    if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6][hh] = v;
  }
  __syncthreads();
  if (threadIdx.x < ATT_HB) {
    float v = -1e30f;
    for (int w = 0; w < ATT_THREADS / 64; ++w) v = (v < wmax[w][threadIdx.x]) ? wmax[w][threadIdx.x] : v;
    smax[threadIdx.x] = v;
  }
  __syncthreads();
  // weights exp8(score - max) (E:820); masked positions and the padding of the whole tiles
  // get weight 0
  for (int idx = threadIdx.x; idx < ATT_HB * NT * ATT_TILE; idx += ATT_THREADS) {
    const int hh = idx / (NT * ATT_TILE), pp = idx - hh * (NT * ATT_TILE);
    sw[hh][pp] = allowed(pb0 + pp) ? exp8(sw[hh][pp] - smax[hh]) : 0.f;
  }
  __syncthreads();
  // sweep 2: o_i = fma chain over positions (E:826-875) straight from the fetched value
  // blocks; value ring slot k holds value tile s = base + k.  A masked or
  // padding position (weight 0) is given value +0: fma(0, 0, o) = o exactly (o is never -0),
  // which is what skipping it in the reference leaves.  The pass's
  // rows are the split's last positions: the register pass leaves them out and they follow
  // from LDS, in position order.  Every wave also forms the l = sum of the weights in
  // position order (E:821) of head wave % ATT_HB (+ 0 leaves the non-negative sum unchanged);
  // waves hh < ATT_HB store theirs.
  const int i = threadIdx.x, wave = threadIdx.x >> 6;
  float o[ATT_HB], lsum = 0.f;
#pragma unroll
  for (int hh = 0; hh < ATT_HB; ++hh) o[hh] = 0.f;
  // a tile every position of which is allowed and none a pass row needs no masks
  const int fa = max(lo_m, c0), fz = min(pos_m, c1 - 1);
  auto full_tile = [=](int pb) {
    return pb >= fa && pb + ATT_TILE - 1 <= fz && (sl_m > sh_m || pb > sh_m || pb + ATT_TILE - 1 < sl_m);
  };
  for (int base = 0; base < NTp; base += ATT_RING)
#pragma unroll
  for (int k = 0; k < ATT_RING; ++k) {
    const int s = base + k;
    const int pb = pb0 + s * ATT_TILE;
    if (s < NT) {  // uniform; otherwise an entry past the split
      const uint32_t vw[16] = {vring[k][0].x, vring[k][0].y, vring[k][0].z, vring[k][0].w,
                               vring[k][1].x, vring[k][1].y, vring[k][1].z, vring[k][1].w,
                               vring[k][2].x, vring[k][2].y, vring[k][2].z, vring[k][2].w,
                               vring[k][3].x, vring[k][3].y, vring[k][3].z, vring[k][3].w};
      const bool full = full_tile(pb);
      const uint32_t keep = full ? 0xFFFFFFFFu : tile_mask(pb);
      // the tile's weights read up front (one LDS round trip per tile instead of one per 4
      // positions); wave w forms head w % ATT_HB's sum from its own copy (no per-head selects)
      float4 w4[ATT_HB][ATT_TILE / 4], wl[ATT_TILE / 4];
#pragma unroll
      for (int p4 = 0; p4 < ATT_TILE / 4; ++p4) {
#pragma unroll
        for (int hh = 0; hh < ATT_HB; ++hh) w4[hh][p4] = *reinterpret_cast<const float4*>(&sw[hh][pb - pb0 + 4 * p4]);
        wl[p4] = *reinterpret_cast<const float4*>(&sw[wave % ATT_HB][pb - pb0 + 4 * p4]);
      }
      auto sweep = [&](const bool masked) {
#pragma unroll
        for (int p4 = 0; p4 < ATT_TILE / 4; ++p4) {
          lsum = (((lsum + wl[p4].x) + wl[p4].y) + wl[p4].z) + wl[p4].w;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int pe = 4 * p4 + q;
            // the position's half word moved to the top (byte select 0x0c gives a zero byte),
            // cleared when masked
            uint32_t vb = __builtin_amdgcn_perm(vw[pe >> 1], vw[pe >> 1], (pe & 1) ? 0x03020c0cu : 0x01000c0cu);
            if (masked) vb &= (uint32_t)((int)(keep << (31 - pe)) >> 31);
            const float vv = as_f32(vb);
#pragma unroll
            for (int hh = 0; hh < ATT_HB; ++hh) {
              const float4 w = w4[hh][p4];
              const float wgt = q == 0 ? w.x : (q == 1 ? w.y : (q == 2 ? w.z : w.w));
              o[hh] = fmaf(wgt, vv, o[hh]);
            }
          }
        }
      };
      if (full) sweep(false);
      else sweep(true);
    }
    // the slot's next entry (past the stream it reloads the last block): every path through
    // the loop issues the same loads, so the wait for a tile never has to cover younger ones
    issue_v(s + ATT_RING, vring[k]);
  }
#pragma unroll
  for (int hh = 0; hh < ATT_HB; ++hh) P.po[(((size_t)t * M + m) * NQ + h0 + hh) * HD + i] = o[hh];
  if ((threadIdx.x & 63) == 0 && wave < ATT_HB) {
    P.pm[((size_t)t * M + m) * NQ + h0 + wave] = smax[wave];
    P.pl[((size_t)t * M + m) * NQ + h0 + wave] = (lo_m > pos_m) ? 0.0f : lsum;
  }
}

// ---- the verify pass's attention: one block per (split t, row m, HB heads) ----
//
// A row of 16 lanes (lane n) holds a 256-vector as the 16 elements e = 16 tt + n, tt = 0..15.
// That is at once the reference's sum-of-squares lane (ss_avx2 accumulator lane n, E:326-345),
// its score chain (s0 lane n for n < 8, s1 lane n - 8 otherwise, E:763-776) and a pair of
// RoPE halves (elements e and e + 128 are tt and tt + 8 of the same lane, E:394-402).  So the
// q/k norm, the rotation and the score of a position each run inside one row, and the rows of
// 16 lanes meet through data-parallel moves instead of LDS round trips and block barriers.  The
// projection writes q, k and v in that order (head16_index), so a lane's 16 values are four
// 16-byte words; the step's RoPE factors and the q/k norm weights are kept in the same order.
constexpr int AR_THREADS = 512;  // 32 rows of 16 lanes; the value sweep: lane = (head, dim)
constexpr int AR_KRING = 6;      // key positions in flight per row of lanes (a sliding-window split: all)
constexpr int AR_HB = 2;         // heads per block: 224 blocks for a 7-row pass
constexpr int AR_VRING = 4;      // value tiles in flight

// E:326-345 1 / sqrtf((float)(ss / 256) + 1e-6) of the row's 256-vector: lane n's double chain
// over tt is accumulator lane n; p_n meet as a_l = (p_l + p_{l+4}) + (p_{l+8} + p_{l+12}),
// ss = (a_0 + a_2) + (a_1 + a_3).  Every lane of the row returns the factor.
__device__ __forceinline__ float row_rms_inv(const float (&x)[16]) {
  double s = 0;
#pragma unroll
  for (int tt = 0; tt < 16; ++tt) {
    const double d = (double)x[tt];
    s = fma(d, d, s);
  }
  const double b = s + shl_d<4>(s);  // lane n: p_n + p_{n+4}
  const double c = b + shl_d<8>(b);  // lanes 0..3: a_l
  const double d = c + shl_d<2>(c);  // lanes 0, 1: a_0 + a_2, a_1 + a_3
  const double e = d + shl_d<1>(d);  // lane 0: ss
  const double ss = bcast0_d(e);
  return 1.0f / sqrtf((float)(ss / HD) + 1e-6f);  // division by a power of two: exact scaling
}

// W:41-44 / E:776 score = hsum8(s0 + s1) of the row's 16 chains (s0 lanes 0..7, s1 lanes 8..15):
// v_j = s0_j + s1_j, then ((v0+v4)+(v1+v5))+((v2+v6)+(v3+v7)), in lane 0 of the row
__device__ __forceinline__ float row_score(float acc) {
  const float u = acc + shl_f<8>(acc);  // lanes 0..7: v_j
  const float w = u + shl_f<4>(u);      // lanes 0..3: v_j + v_{j+4}
  const float z = w + shl_f<1>(w);      // lanes 0, 2: (w0 + w1), (w2 + w3)
  return z + shl_f<2>(z);               // lane 0
}

// E:1307-1324 on one row's 256-vector x held as above: q / k rows r16((x * rinv) * w) rotated
// with the row's factors (cos c[tt], sin s[tt] of elements 16 tt + n, tt < 8)
__device__ __forceinline__ void row_norm_rope(float (&x)[16], const float (&w)[16], const float (&cs)[16]) {
  const float r = row_rms_inv(x);
#pragma unroll
  for (int tt = 0; tt < 16; ++tt) x[tt] = r16((x[tt] * r) * w[tt]);
#pragma unroll
  for (int tt = 0; tt < 8; ++tt) {
    const float u = x[tt], v = x[tt + 8];
    x[tt] = fmaf(u, cs[tt], -(v * cs[8 + tt]));
    x[tt + 8] = fmaf(v, cs[tt], u * cs[8 + tt]);
  }
}

// 16 floats of a lane: four 16-byte words at p
__device__ __forceinline__ void load16(float (&x)[16], const float* p) {
  const float4* p4 = reinterpret_cast<const float4*>(p);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float4 v = p4[k];
    x[4 * k] = v.x;
    x[4 * k + 1] = v.y;
    x[4 * k + 2] = v.z;
    x[4 * k + 3] = v.w;
  }
}

// grid (T, M, NQ / HB): the blocks of split t are t, t + 8, ... in launch order, i.e. all on one
// XCD, whose L2 then fetches the split's key and value tiles once
// The arguments the block needs first lead the list, ahead of the pointer block, so that they
// arrive preloaded in scalar registers (kernel-argument preloading) rather than through a
// dependent load of the argument segment.
// 512 threads: two waves on each SIMD (a wave issues an instruction only every few cycles, so a
// lone wave leaves most of its SIMD idle).  Rows of lanes 0..15 (waves 0-3) form the pass's
// key / value rows while rows 16 + 4 hh (waves 4, 5) form query head hh; 32 rows of lanes score
// positions; in the value sweep thread (hv, i) runs the chain of head hv, dim i.
template <int HB>
__global__ __launch_bounds__(AR_THREADS) void k_attn_rows(const StepDev* __restrict__ sp, const float* __restrict__ q,
                                                          const float* __restrict__ ropestep,
                                                          const float* __restrict__ qnp, const uint16_t* __restrict__ KC,
                                                          const uint16_t* __restrict__ VC, int sliding, int T,
                                                          AttnPtrs P) {
  static_assert(HB * HD == AR_THREADS, "one head per thread in the value sweep");
  constexpr int NR = AR_THREADS / 16;                // rows of 16 lanes
  __shared__ __align__(16) float sw[HB][ATT_SW];     // scores, then weights, of the split's tiles
  __shared__ float rmx[NR][HB];                      // per row of lanes: max of its allowed scores
  __shared__ __align__(16) uint16_t knew[MAXM][HD];  // the pass's key rows, bf16 in cache order
  __shared__ __align__(16) uint16_t vnew[MAXM][HD];  // the pass's value rows, bf16 natural order
  __shared__ __align__(16) float qsh[HB][16][16];    // query head hh, lane n's 16 values at [hh][n]
  const int t = blockIdx.x, m = blockIdx.y, h0 = blockIdx.z * HB;
  const int tid = threadIdx.x, rho = tid >> 4, n = tid & 15, ls = n & 7, ss = n >> 3;
  // 1. loads that need no geometry first: query head qh of the block, its norm weights and the
  // row's RoPE factors, 16 values per lane (head16_index order), for the rows of lanes that form
  // them (rows 16 + 4 qh); the other rows' offsets lie past the resources: they read zeros and
  // move no data.
  const int qh = (rho - 16) >> 2;
  const bool qrow = rho >= 16 && (rho & 3) == 0 && qh < HB;  // uniform per row
  const uint32_t roff = qrow ? (uint32_t)n * 64 : 0x7FFFFFF0u;
  float qx[16], qw[16], cs[16];
  auto load16b = [&](float (&x)[16], __amdgpu_buffer_rsrc_t r, uint32_t off) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint4 v = buf_load16(r, off + 16 * k);
      x[4 * k] = as_f32(v.x);
      x[4 * k + 1] = as_f32(v.y);
      x[4 * k + 2] = as_f32(v.z);
      x[4 * k + 3] = as_f32(v.w);
    }
  };
  {
    const __amdgpu_buffer_rsrc_t rq = buf_rsrc(q + (size_t)m * (NQ * HD) + h0 * HD, HB * HD * 4);
    load16b(qx, rq, qrow ? roff + qh * HD * 4 : roff);
    load16b(qw, buf_rsrc(qnp, HD * 4), roff);
    load16b(cs, buf_rsrc(ropestep + (size_t)m * HD, HD * 4), roff);
  }
  // E:1325-1326 geometry from the step parameters (uniform)
  int rp[MAXM];
#pragma unroll
  for (int r = 0; r < MAXM; ++r) rp[r] = sp->rope[r];
  const int M = sp->M, pos0 = sp->pos0, sl_m = sp->skip_lo[m], sh_m = sp->skip_hi[m], rpm = sp->rope[m];
  const int kmax = pos0 + M - 1;
  int kmin = kmax;
#pragma unroll
  for (int r = 0; r < MAXM; ++r)
    if (r < M) kmin = min(kmin, sliding ? max(0, rp[r] - 511) : 0);
  const int pos_m = pos0 + m, lo_m = sliding ? max(0, rpm - 511) : 0;
  if (m >= M) return;
  const int len = kmax - kmin + 1;
  // (t + 1) len < 2^31 for every launch: 32-bit division
  const int c0 = kmin + (int)((unsigned)(t * len) / (unsigned)T),
            c1 = kmin + (int)((unsigned)((t + 1) * len) / (unsigned)T);
  const int PP = c1 - c0;
  // E:740 attn_allowed for this block's row, restricted to the split
  auto allowed = [=](int p) { return p >= c0 && p < c1 && p >= lo_m && p <= pos_m && !(p >= sl_m && p <= sh_m); };
  auto bits_in = [](int a, int b, int pb) -> uint32_t {  // positions [a, b] within [pb, pb + 31]
    const int lo = max(a - pb, 0), hi = min(b - pb, 31);
    if (lo > hi) return 0u;
    const uint32_t up = hi == 31 ? 0xFFFFFFFFu : ((1u << (hi + 1)) - 1u);
    return up & ~((1u << lo) - 1u);
  };
  auto tile_mask = [=](int pb) -> uint32_t {
    return bits_in(max(lo_m, c0), min(pos_m, c1 - 1), pb) & ~bits_in(sl_m, sh_m, pb);
  };
  const int pb0 = c0 & ~(ATT_TILE - 1);
  const int NT = PP > 0 ? ((c1 - 1) >> 5) - (c0 >> 5) + 1 : 0;
  const int NTp = (NT + AR_VRING - 1) / AR_VRING * AR_VRING;
  // the pass's rows r in [rn0, rn1) have positions pos0 + r inside [c0, c1): the split's last ones
  const int rn0 = max(c0 - pos0, 0), rn1 = min(c1 - pos0, M);

  // 2. the split's first value tiles (lane = dim) and key positions: row rho scores positions
  // c0 + rho + NR k; lane n's 16 key values (slots 32 ls + 16 ss + tt) are two 16-byte words.
  // Keys from the cache stop before pos0 (the pass's rows come from LDS); entries past them
  // read zeros, never used.
  // value tiles: the split's NT blocks of 32 positions from pb0 (entries past them read zeros);
  // lane i reads dim i of a tile, 4 parts of 16 bytes (each load one contiguous 1 KB per wave)
  // the value sweep: wave w's lanes 0..31 run head 0, lanes 32..63 head 1, for dims 32 w + lane % 32;
  // a lane loads the two parts of 8 positions of its dim that its half of the tile holds (head 0's
  // lanes positions 0..15, head 1's 16..31) and the two halves swap them (v_permlane32_swap), so
  // each tile is read once per block for both heads
  const int hv = (tid >> 5) & 1, i = 32 * (tid >> 6) + (tid & 31);
  uint4 vring[AR_VRING][2];
  const __amdgpu_buffer_rsrc_t vrs = buf_rsrc(VC + (size_t)(pb0 >> 5) * (ATT_TILE * HD), (uint32_t)NT * ATT_TILE * HD * 2);
  auto issue_v = [&](int v, uint4 (&r)[2]) {
#pragma unroll
    for (int c = 0; c < 2; ++c)
      r[c] = buf_load16(vrs, (uint32_t)v * (ATT_TILE * HD * 2) + (2 * hv + c) * (8 * HD * 2) + i * 16);
  };
  // key positions below gend = min(c1, pos0) from the cache (the pass's rows come from LDS;
  // entries past gend read zeros, never used)
  const int KN = (PP + NR - 1) / NR, KNp = (KN + AR_KRING - 1) / AR_KRING * AR_KRING;
  const int gend = min(c1, pos0);
  const __amdgpu_buffer_rsrc_t krs = buf_rsrc(KC, (uint32_t)max(gend, 0) * HD * 2);
  uint4 kring[AR_KRING][2];
  auto issue_k = [&](int k, uint4 (&r)[2]) {
    const uint32_t off = (uint32_t)(c0 + rho + NR * k) * (HD * 2) + (4 * ls + 2 * ss) * 16;
    r[0] = buf_load16(krs, off);
    r[1] = buf_load16(krs, off + 16);
  };
#pragma unroll
  for (int k = 0; k < AR_KRING; ++k) issue_k(k, kring[k]);
#pragma unroll
  for (int k = 0; k < AR_VRING; ++k) issue_v(k, vring[k]);

  // 3. E:1307-1324 the pass's key / value rows in this split (rows of lanes 0..7: key row rho,
  // 8..15: value row rho - 8): k = rot(r16((k * rinv) * kn)), v = r16(v * rinv), bf16 into LDS;
  // the block (m 0, h 0) of the split also writes them into the cache.
  // At the same time, 4. the query heads: row 16 + 4 qh forms head qh (E:1307-1324) into LDS.
  if (rn0 < rn1 && rho < 16) {  // uniform per wave
    const int pr = rho & 7;
    const bool prow = pr >= rn0 && pr < rn1;  // uniform per row of lanes
    float px[16];
    if (rho < 8) {  // uniform per wave
      float pw[16], pc[16];
      load16(px, P.kraw + (size_t)pr * HD + 16 * n);
      load16(pw, P.kn + 16 * n);
      load16(pc, ropestep + (size_t)pr * HD + 16 * n);
      row_norm_rope(px, pw, pc);
      if (prow) {
        uint32_t wv[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) wv[k] = (uint32_t)f2bf(px[2 * k]) | ((uint32_t)f2bf(px[2 * k + 1]) << 16);
        uint4* dst = reinterpret_cast<uint4*>(&knew[pr][0]) + 4 * ls + 2 * ss;
        dst[0] = make_uint4(wv[0], wv[1], wv[2], wv[3]);
        dst[1] = make_uint4(wv[4], wv[5], wv[6], wv[7]);
      }
    } else {
      load16(px, P.vraw + (size_t)pr * HD + 16 * n);
      const float r = row_rms_inv(px);
      if (prow) {
#pragma unroll
        for (int tt = 0; tt < 16; ++tt) vnew[pr][16 * tt + n] = f2bf(r16(px[tt] * r));
      }
    }
  }
  if (qrow) {  // uniform per row
    row_norm_rope(qx, qw, cs);
    float4* d4 = reinterpret_cast<float4*>(&qsh[qh][n][0]);
#pragma unroll
    for (int k = 0; k < 4; ++k) d4[k] = make_float4(qx[4 * k], qx[4 * k + 1], qx[4 * k + 2], qx[4 * k + 3]);
  }
  __syncthreads();
  if (rn0 < rn1 && m == 0 && h0 == 0 && tid < HD)
    for (int r = rn0; r < rn1; ++r) {
      P.KCw[(size_t)(pos0 + r) * HD + tid] = knew[r][tid];  // the LDS row is already in cache order
      P.VCw[vc_index(pos0 + r, tid)] = vnew[r][tid];
    }
  float qv[HB][16];  // this lane's query values of the block's heads
#pragma unroll
  for (int hh = 0; hh < HB; ++hh) {
    const float4* s4 = reinterpret_cast<const float4*>(&qsh[hh][n][0]);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float4 v = s4[k];
      qv[hh][4 * k] = v.x;
      qv[hh][4 * k + 1] = v.y;
      qv[hh][4 * k + 2] = v.z;
      qv[hh][4 * k + 3] = v.w;
    }
  }

  // 5. E:750-816 scores of positions c0 + rho + NR k; lane 0 of the row stores them and keeps the
  // running max over the allowed positions (max is order free)
  float rowmax[HB];
#pragma unroll
  for (int hh = 0; hh < HB; ++hh) rowmax[hh] = -1e30f;
  for (int base = 0; base < KNp; base += AR_KRING)
#pragma unroll
    for (int k = 0; k < AR_KRING; ++k) {
      const int kk = base + k;
      if (kk < KN) {  // uniform
        const int p = c0 + rho + NR * kk;
        uint4 ka = kring[k][0], kb = kring[k][1];
        if (c0 + NR * kk + NR - 1 >= pos0) {  // uniform: the step may reach the pass's rows (in LDS)
          const bool own = p >= pos0 && p < c1;
          const uint4* n4 = reinterpret_cast<const uint4*>(&knew[min(max(p - pos0, 0), MAXM - 1)][0]) + 4 * ls + 2 * ss;
          ka = sel4(own, n4[0], ka);
          kb = sel4(own, n4[1], kb);
        }
        const uint32_t kw[8] = {ka.x, ka.y, ka.z, ka.w, kb.x, kb.y, kb.z, kb.w};
        float acc[HB];
#pragma unroll
        for (int hh = 0; hh < HB; ++hh) acc[hh] = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float k0 = as_f32(kw[j] << 16), k1 = as_f32(kw[j] & 0xFFFF0000u);
#pragma unroll
          for (int hh = 0; hh < HB; ++hh) {
            acc[hh] = fmaf(qv[hh][2 * j], k0, acc[hh]);
            acc[hh] = fmaf(qv[hh][2 * j + 1], k1, acc[hh]);
          }
        }
#pragma unroll
        for (int hh = 0; hh < HB; ++hh) {
          const float sc = row_score(acc[hh]);
          if (n == 0 && p < c1) {
            sw[hh][p - pb0] = sc;
            if (allowed(p) && rowmax[hh] < sc) rowmax[hh] = sc;
          }
        }
      }
      issue_k(base + k + AR_KRING, kring[k]);
    }
  if (n == 0)
#pragma unroll
    for (int hh = 0; hh < HB; ++hh) rmx[rho][hh] = rowmax[hh];
  __syncthreads();
  float mx[HB];
#pragma unroll
  for (int hh = 0; hh < HB; ++hh) {
    mx[hh] = -1e30f;
#pragma unroll
    for (int r = 0; r < NR; ++r) mx[hh] = (mx[hh] < rmx[r][hh]) ? rmx[r][hh] : mx[hh];
  }
  // weights exp8(score - max) (E:820); masked positions and the padding of the whole tiles get 0
  for (int idx = tid; idx < HB * NT * ATT_TILE; idx += AR_THREADS) {
    const int hh = idx / (NT * ATT_TILE), pp = idx - hh * (NT * ATT_TILE);
    float mh = mx[0];
#pragma unroll
    for (int k = 1; k < HB; ++k) mh = hh == k ? mx[k] : mh;
    sw[hh][pp] = allowed(pb0 + pp) ? exp8(sw[hh][pp] - mh) : 0.f;
  }
  __syncthreads();

  // 6. E:826-875 o_i = fma chain over the positions in order, lane (hv, i): head hv, dim i; a
  // masked or padding position (weight 0) gets value +0: fma(0, 0, o) = o exactly (o is never
  // -0).  The pass's rows follow from LDS after the tile's other positions (they are the split's
  // last).  Every lane also forms l = the sum of its head's weights in position order (E:821);
  // the lane of head hv, dim 0 (wave 0) stores it.
  float o = 0.f, lsum = 0.f;
  const int fa = max(lo_m, c0), fz = min(min(pos_m, c1 - 1), pos0 - 1);
  auto full_tile = [=](int pb) {
    return pb >= fa && pb + ATT_TILE - 1 <= fz && (sl_m > sh_m || pb > sh_m || pb + ATT_TILE - 1 < sl_m);
  };
  for (int base = 0; base < NTp; base += AR_VRING)
#pragma unroll
    for (int k = 0; k < AR_VRING; ++k) {
      const int s = base + k;
      const int pb = pb0 + s * ATT_TILE;
      if (s < NT) {  // uniform
        // vw[0..7]: parts 0, 1 (positions 0..15) of dim i, vw[8..15]: parts 2, 3; the swap
        // exchanges lanes 32..63 of its first operand with lanes 0..31 of its second
        uint32_t vw[16];
        {
          const uint32_t y[8] = {vring[k][0].x, vring[k][0].y, vring[k][0].z, vring[k][0].w,
                                 vring[k][1].x, vring[k][1].y, vring[k][1].z, vring[k][1].w};
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const auto sw2 = __builtin_amdgcn_permlane32_swap(y[j], y[j], false, false);
            vw[j] = sw2[0];
            vw[8 + j] = sw2[1];
          }
        }
        const bool full = full_tile(pb);
        const uint32_t keep = full ? 0xFFFFFFFFu : tile_mask(pb) & ~bits_in(pos0, pos0 + MAXM, pb);
        // the tile's 32 weights of head hv in every lane of its half wave (LDS broadcast reads):
        // plain VGPR operands, so the two chains need no cross-lane moves (a DPP broadcast
        // operand would also make each chain step wait two instructions for the previous one)
        float wt[ATT_TILE];
        {
          const float4* w4 = reinterpret_cast<const float4*>(&sw[hv][pb - pb0]);
#pragma unroll
          for (int q4 = 0; q4 < ATT_TILE / 4; ++q4) {
            const float4 v = w4[q4];
            wt[4 * q4] = v.x;
            wt[4 * q4 + 1] = v.y;
            wt[4 * q4 + 2] = v.z;
            wt[4 * q4 + 3] = v.w;
          }
        }
        auto sweep = [&](const bool masked) {
#pragma unroll
          for (int pe = 0; pe < ATT_TILE; ++pe) {
            uint32_t vb = __builtin_amdgcn_perm(vw[pe >> 1], vw[pe >> 1], (pe & 1) ? 0x03020c0cu : 0x01000c0cu);
            if (masked) vb &= (uint32_t)((int)(keep << (31 - pe)) >> 31);
            lsum = lsum + wt[pe];
            o = fmaf(wt[pe], as_f32(vb), o);
          }
        };
        if (full) sweep(false);
        else sweep(true);
        if (pb + ATT_TILE > pos0) {  // uniform: the pass's rows in this tile, from LDS
          const int pa = max(max(pb, pos0), c0), pz = min(pb + ATT_TILE, c1);
          for (int pp = pa; pp < pz; ++pp) {
            const float vv = as_f32((uint32_t)vnew[pp - pos0][i] << 16);
            o = fmaf(sw[hv][pp - pb0], vv, o);
          }
        }
      }
      issue_v(s + AR_VRING, vring[k]);
    }
  P.po[(((size_t)t * M + m) * NQ + h0 + hv) * HD + i] = o;
  if (i == 0) {
    P.pm[((size_t)t * M + m) * NQ + h0 + hv] = mx[hv];
    P.pl[((size_t)t * M + m) * NQ + h0 + hv] = (lo_m > pos_m) ? 0.0f : lsum;
  }
}

// E:1019-1059, one block per (row m, head h); M from the geometry or the step parameters
__device__ __forceinline__ void merge_body(const AttnPtrs& P, int M, int T) {
  const int m = blockIdx.x, h = blockIdx.y, i = threadIdx.x;
  // every split's partials are loaded up front (independent loads), then folded in split order
  float pl[MAXT], pm[MAXT], po[MAXT];
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    const size_t k = ((size_t)t * M + m) * NQ + h;
    pl[t] = t < T ? P.pl[k] : 0.f;
    pm[t] = t < T ? P.pm[k] : 0.f;
    po[t] = t < T ? P.po[k * HD + i] : 0.f;
  }
  float M0 = -1e30f;
#pragma unroll
  for (int t = 0; t < MAXT; ++t)
    if (t < T && pl[t] > 0) M0 = (M0 < pm[t]) ? pm[t] : M0;
  double l = 0;
  float acc = 0.f, sc[MAXT];
#pragma unroll
  for (int t = 0; t < MAXT; ++t) {
    sc[t] = 0.f;
    if (t < T && pl[t] > 0) {
      sc[t] = libm_expf_neg(pm[t] - M0, c_expf_tab);
      l = fma((double)pl[t], (double)sc[t], l);
    }
  }
  const float inv = (float)(1.0 / l);
#pragma unroll
  for (int t = 0; t < MAXT; ++t)
    if (t < T && pl[t] > 0) acc = fmaf(po[t], sc[t], acc);
  const float y = r16(acc * inv);
  if (!P.gs) {
    P.out[(size_t)m * P.ldo + h * HD + i] = y;
    return;
  }
  // the head's 256 outputs are the 8 groups 8h..8h+7 of the o_proj input: staged copy + sums
  __shared__ __align__(16) float ys[HD];
  ys[i] = y;
  __syncthreads();
  float* xs = P.out + (size_t)m * P.ldo + h * HD;
  if (i < HD / 4) {
    const float* b = ys + (i >> 3) * 32;
    const int j = i & 7;
    reinterpret_cast<float4*>(xs)[i] = make_float4(b[2 * j], b[16 + 2 * j], b[2 * j + 1], b[17 + 2 * j]);
  }
  if (i < HD / 32) {
    const float4* b4 = reinterpret_cast<const float4*>(ys + i * 32);
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float4 r = b4[k];
      s = (((s + r.x) + r.y) + r.z) + r.w;
    }
    P.gs[(size_t)m * (P.ldo / 32) + h * (HD / 32) + i] = s;
  }
  if (P.xq && i < HD / 32) {  // the head's 8 groups of the row, one a thread (ys in plain order)
    float v[32];
#pragma unroll
    for (int k = 0; k < 32; ++k) v[k] = ys[i * 32 + k];
    uint64_t q[4];
    const size_t gq = (size_t)m * (P.ldo / 32) + h * (HD / 32) + i;
    P.xqs[gq] = a8_quant_group(v, q);
#pragma unroll
    for (int hw = 0; hw < 4; ++hw) P.xq[gq * 4 + hw] = q[hw];
  }
}

__global__ __launch_bounds__(HD) void k_attn_merge(AttnPtrs P, int M, int T) { merge_body(P, M, T); }

void launch_attn(uint16_t* KC, uint16_t* VC, const float* q, const float* k, const float* v, const LayerNorms& ln,
                 const float* ropestep, const StepDev* sp, int sliding, int T, float* po, float* pm, float* pl, int M,
                 hipStream_t st) {
  AttnPtrs P{KC, VC, q, NQ * HD, po, pm, pl, nullptr, NQ * HD, nullptr, k, v, ropestep, ln.qnp, ln.knp, KC, VC};
  hipLaunchKernelGGL(k_attn_rows<AR_HB>, dim3(T, M, NQ / AR_HB), dim3(AR_THREADS), 0, st, sp, q, ropestep, ln.qnp,
                     (const uint16_t*)KC, (const uint16_t*)VC, sliding, T, P);
}

void launch_attn_merge(const float* po, const float* pm, const float* pl, int M, int T, float* out, int ldo,
                       float* gs, hipStream_t st, uint64_t* xq, float* xqs) {
  AttnPtrs P{nullptr, nullptr, nullptr, 0, const_cast<float*>(po), const_cast<float*>(pm), const_cast<float*>(pl),
             out, ldo, gs, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, xq, xqs};
  hipLaunchKernelGGL(k_attn_merge, dim3(M, NQ), dim3(HD), 0, st, P, M, T);
}

void launch_attn_geom(const uint16_t* KC, const uint16_t* VC, const float* q, int ldq, const AttnGeom& g,
                      float* po, float* pm, float* pl, float* out, int ldo, hipStream_t st, int nh, float* gs) {
  AttnPtrs P{KC, VC, q, ldq, po, pm, pl, out, ldo, gs, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
             nullptr};
  hipLaunchKernelGGL(k_attn_split, dim3(g.T, g.M, nh / ATT_HB), dim3(ATT_THREADS), 0, st, P, g, g.T);
  hipLaunchKernelGGL(k_attn_merge, dim3(g.M, nh), dim3(HD), 0, st, P, g.M, g.T);
}

void launch_attn_geom_dev(const uint16_t* KC, const uint16_t* VC, const float* q, int ldq, const AttnGeom* gdev, int M,
                          int T, float* po, float* pm, float* pl, float* out, int ldo, hipStream_t st, int nh,
                          float* gs, uint64_t* xq, float* xqs) {
  AttnPtrs P{KC, VC, q, ldq, po, pm, pl, out, ldo, gs, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
             nullptr, gdev, xq, xqs};
  AttnGeom g{};
  g.M = M;
  g.T = T;
  hipLaunchKernelGGL(k_attn_split, dim3(T, M, nh / ATT_HB), dim3(ATT_THREADS), 0, st, P, g, T);
  hipLaunchKernelGGL(k_attn_merge, dim3(M, nh), dim3(HD), 0, st, P, M, T);
}

// E:1325-1326 per layer type: keys [kmin, pos0 + M - 1], row m at slot pos0 + m with its window
// from its RoPE position (sliding: 512 keys) and the step's skipped range
__global__ void k_step_geom(const StepDev* __restrict__ sp, int T, AttnGeom* __restrict__ geo) {
  const int ty = threadIdx.x;  // 0 sliding, 1 global
  if (ty > 1) return;
  AttnGeom g{};
  const int M = sp->M, pos0 = sp->pos0;
  g.M = M;
  g.T = T;
  g.kmax = pos0 + M - 1;
  g.kmin = g.kmax;
  for (int m = 0; m < MAXM; ++m) {
    if (m >= M) break;
    g.pos[m] = pos0 + m;
    g.lo[m] = ty == 0 ? max(0, sp->rope[m] - 511) : 0;
    g.skip_lo[m] = sp->skip_lo[m];
    g.skip_hi[m] = sp->skip_hi[m];
    g.kmin = min(g.kmin, g.lo[m]);
  }
  geo[ty] = g;
}
void launch_step_geom(const StepDev* sp, int T, AttnGeom* geo, hipStream_t st) {
  hipLaunchKernelGGL(k_step_geom, dim3(1), dim3(64), 0, st, sp, T, geo);
}

// the caller's [position][256] key / value rows (device) into the device cache layout
// (kc_index / vc_index), positions npos .. kv_cap(npos) - 1 zero
__global__ void k_kv_to_cache(const uint16_t* __restrict__ K, const uint16_t* __restrict__ V, int npos,
                              uint16_t* __restrict__ KC, uint16_t* __restrict__ VC) {
  const size_t total = (size_t)((npos + 31) / 32 * 32) * HD;
  for (size_t u = (size_t)blockIdx.x * blockDim.x + threadIdx.x; u < total; u += (size_t)gridDim.x * blockDim.x) {
    const int p = (int)(u / HD), e = (int)(u % HD);
    KC[kc_index(p, e)] = p < npos ? K[u] : (uint16_t)0;
    VC[vc_index(p, e)] = p < npos ? V[u] : (uint16_t)0;
  }
}

void launch_kv_to_cache(const uint16_t* K, const uint16_t* V, int npos, uint16_t* KC, uint16_t* VC, hipStream_t st) {
  const size_t total = (size_t)kv_cap(npos) * HD;
  int grid = (int)((total + 255) / 256);
  if (grid > 4096) grid = 4096;
  hipLaunchKernelGGL(k_kv_to_cache, dim3(grid), dim3(256), 0, st, K, V, npos, KC, VC);
}

int attn_pmax() { return ATT_PMAX; }

}  // namespace g4v
