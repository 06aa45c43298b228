// g4v_attn.hip -- split-KV attention over the draft rows (E:743-877) and the exact
// log-sum-exp merge of the splits (E:1019-1059), gfx950.  E = engine/gemma4_engine.cpp.
//
// Split t covers keys [kmin + t*len/T, kmin + (t+1)*len/T) exactly as the reference's
// worker t does, and every per-(row, head) value is produced in the reference's fp32 order:
//   score_p = hsum8(s0 + s1), s0/s1 two 8-lane FMA chains over the head dim in steps of 16;
//   w_p = exp8(score_p - max), l = sum of w_p in position order, o_i = fma chain over p;
//   merge: sc_t = libm expf(max_t - M0), l = sum_t (double) l_t sc_t,
//          out = r16((fma chain over splits of o_t sc_t) * (float)(1 / l)).
// One block serves (split t, row m, ATT_HB heads): the block's K/V rows are staged through LDS
// tile by tile (the next tile is fetched into registers while the current one is used) and
// shared by the block's heads.
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
  const float* qn;    // q_norm / k_norm weights [HD]
  const float* kn;
  uint16_t* KCw;      // the layer's cache (same as KC / VC), written for the pass's rows
  uint16_t* VCw;
  const AttnGeom* gdev;  // raw attention: the geometry in device memory (replaces the argument)
};

// E:326-345 sum of squares of a 256-vector, 16 lanes x 16 steps in double, combined in the
// reference's order; part[t] = lane t's sum (t < 16).  Returns 1 / sqrtf((float)(ss / n) + 1e-6).
__device__ __forceinline__ float rms_inv16(const double* part) {
  double a[4];
#pragma unroll
  for (int l = 0; l < 4; ++l) a[l] = (part[l] + part[4 + l]) + (part[8 + l] + part[12 + l]);
  const double ss = (a[0] + a[2]) + (a[1] + a[3]);
  return 1.0f / sqrtf((float)(ss / HD) + 1e-6f);  // division by a power of two: exact scaling
}

// grid (T, M, NQ / ATT_HB)
template <bool STEP>
__global__ __launch_bounds__(ATT_THREADS) void k_attn_split(AttnPtrs P, AttnGeom gin, const StepDev* sp, int sliding,
                                                            int T) {
  __shared__ float qs[ATT_HB][8][32];              // lane l's 32 query values: s0 chain then s1 chain
  __shared__ __align__(16) float sw[ATT_HB][ATT_SW];
  __shared__ float wmax[ATT_THREADS / 64][ATT_HB];
  __shared__ float smax[ATT_HB];
  // verify pass: rows being normalised (the block's query heads, then the pass's k and v rows),
  // their 16-lane partial sums of squares, and the pass's finished key rows (bf16, in the
  // key cache's chain-lane order) and value rows (bf16, natural order)
  __shared__ float nx[STEP ? ATT_HB + 2 * MAXM : 1][HD];
  __shared__ double npart[STEP ? ATT_HB + 2 * MAXM : 1][16];
  __shared__ float nrinv[STEP ? ATT_HB + 2 * MAXM : 1];
  __shared__ __align__(16) uint16_t knew[STEP ? MAXM : 1][HD];
  __shared__ __align__(16) uint16_t vnew[STEP ? MAXM : 1][HD];
  const int t = blockIdx.x, m = blockIdx.y, h0 = blockIdx.z * ATT_HB;
  const int e = threadIdx.x;  // element e: chain s = (e/8)%2, step tt = e/16, lane e%8
  const int i2 = e & (HD / 2 - 1);
  // Every load that does not depend on the step geometry is issued first, together with the
  // geometry itself (one round trip): the query heads and, in a verify pass, their norm weights
  // and RoPE factors.  The pass's raw key/value rows are the context's last positions: the last
  // two splits load them (and their RoPE factors) up front, any other split only when the
  // geometry puts some of them in it (a context shorter than T rows per split).
  float qv[ATT_HB];
#pragma unroll
  for (int hh = 0; hh < ATT_HB; ++hh) qv[hh] = P.q[(size_t)m * P.ldq + (h0 + hh) * HD + e];
  float kv[2][MAXM] = {}, ck[MAXM] = {}, sk[MAXM] = {}, qw = 0.f, kw = 0.f, cq = 0.f, sq = 0.f;
  auto load_rows = [&]() {
#pragma unroll
    for (int r = 0; r < MAXM; ++r) {
      kv[0][r] = P.kraw[(size_t)r * HD + e];
      kv[1][r] = P.vraw[(size_t)r * HD + e];
      ck[r] = P.ropestep[(size_t)r * HD + i2];
      sk[r] = P.ropestep[(size_t)r * HD + HD / 2 + i2];
    }
  };
  if (STEP) {
    qw = P.qn[e];
    kw = P.kn[e];
    cq = P.ropestep[(size_t)m * HD + i2];
    sq = P.ropestep[(size_t)m * HD + HD / 2 + i2];
    if (t >= T - 2) load_rows();
  }
  // E:1325-1326 geometry: every thread reads the (uniform) parameters itself, no serial set-up;
  // all fields are read unconditionally so that they arrive together
  int M, kmin, kmax, lo_m, pos_m, sl_m, sh_m, pos0 = 0;
  if (STEP) {
    int rp[MAXM];
#pragma unroll
    for (int r = 0; r < MAXM; ++r) rp[r] = sp->rope[r];
    const int rpm = sp->rope[m];
    M = sp->M;
    pos0 = sp->pos0;
    sl_m = sp->skip_lo[m];
    sh_m = sp->skip_hi[m];
    kmax = pos0 + M - 1;
    kmin = kmax;
#pragma unroll
    for (int r = 0; r < MAXM; ++r)
      if (r < M) kmin = min(kmin, sliding ? max(0, rp[r] - 511) : 0);
    pos_m = pos0 + m;
    lo_m = sliding ? max(0, rpm - 511) : 0;
  } else {
    const AttnGeom& G = P.gdev ? *P.gdev : gin;
    M = G.M;
    kmin = G.kmin;
    kmax = G.kmax;
    pos_m = G.pos[m];
    lo_m = G.lo[m];
    sl_m = G.skip_lo[m];
    sh_m = G.skip_hi[m];
  }
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
  // the split); value tile: lane i takes dim i of the block's 32 positions (64 bytes)
  // Every stream entry issues its four loads, so each ring slot has exactly one definition
  // per tile (no merges that would make the compiler wait on loads still in flight): empty
  // entries and entries past the stream load a row they never use.
  uint4 kring[ATT_RING][4], vring[ATT_RING][4];
  const uint16_t* kbase = P.KC + l * 32;
  const uint16_t* vbase = P.VC + threadIdx.x * 32;
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
    for (int c = 0; c < 4; ++c) r[c] = src[c];
  };
  // the pass's rows r in [rn0, rn1) have positions pos0 + r inside [c0, c1); they are the
  // split's last positions
  const int rn0 = STEP ? max(c0 - pos0, 0) : 0, rn1 = STEP ? min(c1 - pos0, M) : 0;
  if (STEP && t < T - 2 && rn0 < rn1) load_rows();
  __builtin_amdgcn_sched_barrier(0);  // keep the prologue loads ahead of the tile loads
  // the key tiles now (also when the split is empty: no paths with fewer loads in flight); the
  // value tiles once the pass's rows have arrived, so that they do not queue in front of them
#pragma unroll
  for (int k = 0; k < ATT_RING; ++k) issue_k(k, kring[k]);
  __builtin_amdgcn_sched_barrier(0);
  if (STEP) {
    // E:1307-1324 on the block's query heads and the pass's key/value rows of this split:
    // x = r16((x * rms_inv) * w) (v: r16(x * rms_inv)), then NeoX rotation of q and k
#pragma unroll
    for (int hh = 0; hh < ATT_HB; ++hh) nx[hh][e] = qv[hh];
#pragma unroll
    for (int r = 0; r < MAXM; ++r)
      if (r >= rn0 && r < rn1) {  // uniform
        nx[ATT_HB + r][e] = kv[0][r];
        nx[ATT_HB + MAXM + r][e] = kv[1][r];
      }
    __syncthreads();
    for (int idx = threadIdx.x; idx < (ATT_HB + 2 * MAXM) * 16; idx += ATT_THREADS) {
      const int row = idx >> 4, t16 = idx & 15;
      const bool live = row < ATT_HB || ((row - ATT_HB) % MAXM >= rn0 && (row - ATT_HB) % MAXM < rn1);
      double sacc = 0;
      if (live) {
#pragma unroll
        for (int k = 0; k < 16; ++k) {
          const double d = (double)nx[row][16 * k + t16];
          sacc = fma(d, d, sacc);
        }
      }
      npart[row][t16] = sacc;
    }
    __syncthreads();
    if (threadIdx.x < ATT_HB + 2 * MAXM) nrinv[threadIdx.x] = rms_inv16(npart[threadIdx.x]);  // once per row
    __syncthreads();
#pragma unroll
    for (int hh = 0; hh < ATT_HB; ++hh) nx[hh][e] = r16((qv[hh] * nrinv[hh]) * qw);
#pragma unroll
    for (int r = 0; r < MAXM; ++r)
      if (r >= rn0 && r < rn1) {  // uniform
        nx[ATT_HB + r][e] = r16((kv[0][r] * nrinv[ATT_HB + r]) * kw);
        vnew[r][e] = f2bf(r16(kv[1][r] * nrinv[ATT_HB + MAXM + r]));
      }
    __syncthreads();
    // E:394-402 NeoX halves: out_i = fma(u, c, -(w s)) and out_{i+128} = fma(w, c, u s)
    auto rot = [&](const float* y, float c, float sn) {
      return e < HD / 2 ? fmaf(y[e], c, -(y[e + HD / 2] * sn)) : fmaf(y[e], c, y[e - HD / 2] * sn);
    };
#pragma unroll
    for (int hh = 0; hh < ATT_HB; ++hh) qv[hh] = rot(nx[hh], cq, sq);
#pragma unroll
    for (int r = 0; r < MAXM; ++r)
      if (r >= rn0 && r < rn1) knew[r][kc_slot(e)] = f2bf(rot(nx[ATT_HB + r], ck[r], sk[r]));
    __syncthreads();
    if (m == 0 && h0 == 0)  // one block per split writes the pass's rows that fall in it
      for (int r = rn0; r < rn1; ++r) {
        P.KCw[(size_t)(pos0 + r) * HD + e] = knew[r][e];  // the LDS row is already in cache order
        P.VCw[vc_index(pos0 + r, e)] = vnew[r][e];
      }
  }
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
      if (STEP && pb + ATT_TILE > pos0) {  // uniform: the tile may hold rows of the pass (in LDS)
        const bool own = p >= pos0 && p < c1;
        const uint4* n4 = reinterpret_cast<const uint4*>(&knew[min(max(p - pos0, 0), MAXM - 1)][l * 32]);
#pragma unroll
        for (int c = 0; c < 4; ++c) kr[c] = sel4(own, n4[c], kr[c]);
      }
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
  const int fa = max(lo_m, c0), fz = min(min(pos_m, c1 - 1), STEP ? pos0 - 1 : 0x7fffffff);
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
      const uint32_t keep = full ? 0xFFFFFFFFu : tile_mask(pb) & (STEP ? ~bits_in(pos0, pos0 + MAXM, pb) : 0xFFFFFFFFu);
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
      if (STEP && pb + ATT_TILE > pos0) {  // uniform: the pass's rows in this tile, from LDS
        const int pa = max(max(pb, pos0), c0), pz = min(pb + ATT_TILE, c1);
        for (int pp = pa; pp < pz; ++pp) {
          const float vv = as_f32((uint32_t)vnew[pp - pos0][i] << 16);
#pragma unroll
          for (int hh = 0; hh < ATT_HB; ++hh) o[hh] = fmaf(sw[hh][pp - pb0], vv, o[hh]);
        }
      }
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
}

__global__ __launch_bounds__(HD) void k_attn_merge(AttnPtrs P, int M, int T) { merge_body(P, M, T); }

void launch_attn(uint16_t* KC, uint16_t* VC, const float* q, const float* k, const float* v, const LayerNorms& ln,
                 const float* ropestep, const StepDev* sp, int sliding, int T, float* po, float* pm, float* pl, int M,
                 hipStream_t st) {
  AttnPtrs P{KC, VC, q, NQ * HD, po, pm, pl, nullptr, NQ * HD, nullptr, k, v, ropestep, ln.qn, ln.kn, KC, VC};
  AttnGeom g{};
  hipLaunchKernelGGL(k_attn_split<true>, dim3(T, M, NQ / ATT_HB), dim3(ATT_THREADS), 0, st, P, g, sp, sliding, T);
}

void launch_attn_geom(const uint16_t* KC, const uint16_t* VC, const float* q, int ldq, const AttnGeom& g,
                      float* po, float* pm, float* pl, float* out, int ldo, hipStream_t st, int nh, float* gs) {
  AttnPtrs P{KC, VC, q, ldq, po, pm, pl, out, ldo, gs, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
             nullptr};
  hipLaunchKernelGGL(k_attn_split<false>, dim3(g.T, g.M, nh / ATT_HB), dim3(ATT_THREADS), 0, st, P, g,
                     (const StepDev*)nullptr, 0, g.T);
  hipLaunchKernelGGL(k_attn_merge, dim3(g.M, nh), dim3(HD), 0, st, P, g.M, g.T);
}

void launch_attn_geom_dev(const uint16_t* KC, const uint16_t* VC, const float* q, int ldq, const AttnGeom* gdev, int M,
                          int T, float* po, float* pm, float* pl, float* out, int ldo, hipStream_t st, int nh) {
  AttnPtrs P{KC, VC, q, ldq, po, pm, pl, out, ldo, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
             nullptr, gdev};
  AttnGeom g{};
  g.M = M;
  g.T = T;
  hipLaunchKernelGGL(k_attn_split<false>, dim3(T, M, nh / ATT_HB), dim3(ATT_THREADS), 0, st, P, g,
                     (const StepDev*)nullptr, 0, T);
  hipLaunchKernelGGL(k_attn_merge, dim3(M, nh), dim3(HD), 0, st, P, M, T);
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
