// g4v_attn_hd.hip -- split-KV attention (E:743-877) and its merge (E:1019-1059) for a head dim
// D other than 256: the 512-wide global layers of the Gemma-4-E2B layout.  Same arithmetic as
// g4v_attn.hip, in a plainer form (global layers are one in five):
//   split t covers keys [kmin + t len / T, kmin + (t + 1) len / T);
//   score_p = hsum8(s0 + s1), s0 / s1 the two 8-lane FMA chains over the head dim in steps of
//     16 (lane l, chain s: elements 16 tt + 8 s + l in tt order);
//   w_p = exp8(score_p - max) over the allowed positions; l = sum of w_p in position order;
//     o_i = fma chain of w_p v_p,i in position order (disallowed positions skipped);
//   merge: sc_t = libm expf(max_t - M0), l = sum_t (double) l_t sc_t,
//     out = r16((fma chain over splits of o_t sc_t) * (float)(1 / l)).
// One block per (split, row, head); q rows arrive normalised and rotated (k_pf_qkv).
#include "g4v_layer.h"

namespace g4v {

__constant__ uint64_t c_expf_tab_hd[32] = G4V_EXPF_TABLE;

// geometry from the launch (gv) or, when gp is given, from device memory (a drafter chain's steps);
// D threads: 8 lanes per position for the scores, one output dim per thread for the values.
// Scores and weights live in sw indexed from pa, the 8-aligned position at or below c0, so that
// the value pass reads 8 positions of its dim (16 bytes of the cache) and 8 weights at a time.
template <int D>
__global__ __launch_bounds__(D) void k_attn_split_d(const uint16_t* __restrict__ KC, const uint16_t* __restrict__ VC,
                                                   const float* __restrict__ q, int ldq, AttnGeom gv,
                                                   const AttnGeom* __restrict__ gp, float* __restrict__ po,
                                                   float* __restrict__ pm, float* __restrict__ pl) {
  constexpr int NTH = D;
  const AttnGeom& g = gp ? *gp : gv;
  __shared__ __align__(16) float qs[D];                   // the head's query in key-slot order
  constexpr int SW_PAD = ATT_SPLIT_MAX + 80;  // slots [0, SW_PAD): scores, then weights, from pa
  __shared__ __align__(16) float sw[SW_PAD + 64];
  __shared__ float red[NTH / 64];
  const int t = blockIdx.x, m = blockIdx.y, h = blockIdx.z, T = g.T;
  const int M = g.M;
  if (m >= M) return;  // uniform
  const int len = g.kmax - g.kmin + 1;
  // (uniform; readfirstlane says so, so that the loops below count in scalar registers)
  const int c0 = __builtin_amdgcn_readfirstlane(g.kmin + (int)((long)t * len / T));
  const int c1 = __builtin_amdgcn_readfirstlane(g.kmin + (int)((long)(t + 1) * len / T));
  const int pa = c0 & ~7, pe = (c1 + 7) & ~7;
  const int lo = g.lo[m], pos = g.pos[m], sl = g.skip_lo[m], sh = g.skip_hi[m];
  auto allowed = [=](int p) { return p >= lo && p <= pos && !(p >= sl && p <= sh); };  // E:740
  for (int e = threadIdx.x; e < D; e += NTH) qs[kc_slot_d<D>(e)] = q[(size_t)m * ldq + h * D + e];
  __syncthreads();
  // scores: 8 lanes per position, NP = NTH / 8 positions per pass, the key words of KR passes in
  // flight.  The keys are read through a resource over rows [0, c1): a lane past c1 reads zeros
  // and its score is not stored, so the ring runs without branches (a pass past the split only
  // computes)
  const int ps = threadIdx.x >> 3, l = threadIdx.x & 7;
  constexpr int KW = D / 64, NP = NTH / 8, KR = 4;  // uint4 of a key row per lane (two chains)
  const __amdgpu_buffer_rsrc_t krs = buf_rsrc(KC, (uint32_t)c1 * (D * 2));
  static_assert(D == 512, "the key slot layout read here is kc_slot_d<512>'s");
  // lane l's word k (chain k / 4, steps 8 (k % 4) .. + 7) is 16-byte word 8 k + l of the row
  auto load_k = [&](int p0, uint4 (&kk)[KW]) {
    const uint32_t off = (uint32_t)(p0 + ps) * (D * 2) + l * 16;
#pragma unroll
    for (int k = 0; k < KW; ++k) kk[k] = buf_load16(krs, off + k * 128);
  };
  auto score = [&](int p0, const uint4 (&kk)[KW]) {
    float s[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      float a = 0.f;
#pragma unroll
      for (int tt = 0; tt < D / 16; tt += 8) {
        const uint4 k4 = kk[c * (D / 128) + tt / 8];
        const uint32_t kw[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {  // the query in the same slots: kc_slot_d of step tt + 2 k (+ 1)
          a = fmaf(qs[64 * (4 * c + tt / 8) + 8 * l + 2 * k], as_f32(kw[k] << 16), a);
          a = fmaf(qs[64 * (4 * c + tt / 8) + 8 * l + 2 * k + 1], as_f32(kw[k] & 0xFFFF0000u), a);
        }
      }
      s[c] = a;
    }
    const float v = hsum8_lanes(s[0] + s[1]);
    // lane 0 of a position's 8 holds its score; the other lanes and the positions past c1 write
    // pad slots past every slot read (no branch in the ring's loop)
    sw[(l == 0 && p0 + ps < c1) ? p0 + ps - pa : SW_PAD + (threadIdx.x & 63)] = v;
  };
  uint4 kr[KR][KW];
#pragma unroll
  for (int i = 0; i < KR; ++i) {  // in slot order, as the loop reloads them
    load_k(c0 + i * NP, kr[i]);
    __builtin_amdgcn_sched_barrier(0);
  }
  for (int p0 = c0; p0 < c1; p0 += KR * NP) {
#pragma unroll
    for (int i = 0; i < KR; ++i) {
      score(p0 + i * NP, kr[i]);
      __builtin_amdgcn_sched_barrier(0);  // the slot is used before its next load
      load_k(p0 + (i + KR) * NP, kr[i]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __syncthreads();
  // the max over the allowed positions (order free)
  float mx = -1e30f;
  for (int p = c0 + threadIdx.x; p < c1; p += NTH)
    if (allowed(p)) mx = fmaxf(mx, sw[p - pa]);
  for (int s = 1; s < 64; s <<= 1) mx = fmaxf(mx, __shfl_xor(mx, s, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = red[0];
#pragma unroll
  for (int w = 1; w < NTH / 64; ++w) mx = fmaxf(mx, red[w]);
  // weights exp8(score - max) of the allowed positions (E:820), 0 for every other slot of
  // [pa, pa + 8 nv); each thread rewrites only the slots it reads
  constexpr int VR = 8;  // value steps in flight
  const int n8 = (pe - pa) / 8, nv = (n8 + VR - 1) / VR * VR;  // 8 nv <= ATT_SPLIT_MAX + 69
  for (int j = threadIdx.x; j < 8 * nv; j += NTH) {
    const int p = pa + j;
    sw[j] = (p >= c0 && p < c1 && allowed(p)) ? exp8(sw[j] - mx) : 0.f;
  }
  __syncthreads();
  // o_d = fma chain over the positions in order (E:821-875), l = the weights' sum in order;
  // a zero weight (not allowed, outside the split) leaves both unchanged: its value is taken
  // as +0 and o is never -0
  const int d = threadIdx.x;
  float o = 0.f, lsum = 0.f;
  // the value words of 8 positions of dim d (16 contiguous bytes of the cache), VR steps in
  // flight with no branch between a load and its use, through a resource over the cache parts
  // of 32 positions up to the one holding pe - 1 (within the slab); the steps past n8 weigh 0
  const __amdgpu_buffer_rsrc_t vrs = buf_rsrc(VC, (uint32_t)(((pe - 1) >> 5) + 1) * (32 * D * 2));
  auto load_v = [&](int j) {
    const int p8 = pa + 8 * j;
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
      const uint32_t u4[4] = {ring[i].x, ring[i].y, ring[i].z, ring[i].w};
      float v8[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) v8[k] = as_f32((k & 1) ? (u4[k >> 1] & 0xFFFF0000u) : (u4[k >> 1] << 16));
      __builtin_amdgcn_sched_barrier(0);
      ring[i] = load_v(jb + VR + i);
      __builtin_amdgcn_sched_barrier(0);
      const int j8 = 8 * (jb + i);
      const float4 wa = *reinterpret_cast<const float4*>(&sw[j8]);
      const float4 wb = *reinterpret_cast<const float4*>(&sw[j8 + 4]);
      const float w8[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const float vv = w8[k] != 0.f ? v8[k] : 0.f;
        o = fmaf(w8[k], vv, o);
        lsum = lsum + w8[k];
      }
    }
  }
  const size_t k = ((size_t)t * M + m) * NQ + h;
  po[k * D + d] = o;
  if (threadIdx.x == 0) {
    pm[k] = mx;
    pl[k] = lsum;  // 0 when the split holds no allowed position: the merge then skips it
  }
}

// E:1019-1059, one block per (row m, head h), one thread per dim; out staged (the o-projection
// input, staged_index) with its group sums when gs is given, else plain [M][ldo]; with gs and xq,
// the rows also quantised for a W4A8 product (words of group g of row m at xq[(m ldo / 32 + g) 4])
template <int D>
__global__ __launch_bounds__(D) void k_attn_merge_d(const float* __restrict__ po, const float* __restrict__ pm,
                                                    const float* __restrict__ pl, int M, int T, float* __restrict__ out,
                                                    int ldo, float* __restrict__ gs, uint64_t* __restrict__ xq,
                                                    float* __restrict__ xqs) {
  __shared__ __align__(16) float ys[D];
  const int m = blockIdx.x, h = blockIdx.y, i = threadIdx.x;
  float M0 = -1e30f;
  for (int t = 0; t < T; ++t) {
    const size_t k = ((size_t)t * M + m) * NQ + h;
    if (pl[k] > 0) M0 = (M0 < pm[k]) ? pm[k] : M0;
  }
  double l = 0;
  float acc = 0.f;
  for (int t = 0; t < T; ++t) {
    const size_t k = ((size_t)t * M + m) * NQ + h;
    if (pl[k] > 0) {
      const float sc = libm_expf_neg(pm[k] - M0, c_expf_tab_hd);
      l = fma((double)pl[k], (double)sc, l);
      acc = fmaf(po[k * D + i], sc, acc);
    }
  }
  const float y = r16(acc * (float)(1.0 / l));
  if (!gs) {
    out[(size_t)m * ldo + h * D + i] = y;
    return;
  }
  ys[i] = y;
  __syncthreads();
  float* xs = out + (size_t)m * ldo + h * D;
  if (i < D / 4) {  // float4 index 8 g + j of the head's groups g (staged_index)
    const float* b = ys + (i >> 3) * 32;
    const int j = i & 7;
    reinterpret_cast<float4*>(xs)[i] = make_float4(b[2 * j], b[16 + 2 * j], b[2 * j + 1], b[17 + 2 * j]);
  }
  if (i < D / 32) {
    const float4* b4 = reinterpret_cast<const float4*>(ys + i * 32);
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float4 r = b4[k];
      s = (((s + r.x) + r.y) + r.z) + r.w;
    }
    gs[(size_t)m * (ldo / 32) + h * (D / 32) + i] = s;
  }
  if (xq && i < D / 32) {  // engine/w4a8_avx2.h:33-41 on the head's groups (ys in plain order)
    float v[32];
#pragma unroll
    for (int k = 0; k < 32; ++k) v[k] = ys[i * 32 + k];
    uint64_t q[4];
    const size_t gq = (size_t)m * (ldo / 32) + h * (D / 32) + i;
    xqs[gq] = a8_quant_group(v, q);
#pragma unroll
    for (int hw = 0; hw < 4; ++hw) xq[gq * 4 + hw] = q[hw];
  }
}

int launch_attn_geom_hd(const uint16_t* KC, const uint16_t* VC, const float* q, int ldq, const AttnGeom& g, int hd,
                        float* po, float* pm, float* pl, float* out, int ldo, float* gs, hipStream_t st) {
  if (hd != 512 || g.M < 1 || g.M > MAXM || g.T < 1 || g.T > MAXT) return -1;
  const int len = g.kmax - g.kmin + 1;
  if (len < 1 || (len + g.T - 1) / g.T + 1 > ATT_SPLIT_MAX) return -1;
  hipLaunchKernelGGL(k_attn_split_d<512>, dim3(g.T, g.M, NQ), dim3(512), 0, st, KC, VC, q, ldq, g,
                     (const AttnGeom*)nullptr, po, pm, pl);
  hipLaunchKernelGGL(k_attn_merge_d<512>, dim3(g.M, NQ), dim3(512), 0, st, po, pm, pl, g.M, g.T, out, ldo, gs,
                     (uint64_t*)nullptr, (float*)nullptr);
  return 0;
}

void launch_attn_geom_dev_hd(const uint16_t* KC, const uint16_t* VC, const float* q, int ldq, const AttnGeom* gdev,
                             int M, int T, int nh, float* po, float* pm, float* pl, float* out, int ldo, hipStream_t st,
                             float* gs, uint64_t* xq, float* xqs) {
  AttnGeom g{};
  g.M = M;
  g.T = T;
  hipLaunchKernelGGL(k_attn_split_d<512>, dim3(T, M, nh), dim3(512), 0, st, KC, VC, q, ldq, g, gdev, po, pm, pl);
  hipLaunchKernelGGL(k_attn_merge_d<512>, dim3(M, nh), dim3(512), 0, st, po, pm, pl, M, T, out, ldo, gs, xq, xqs);
}

}  // namespace g4v
