// g4v_num.h -- scalar numerics shared by the gfx950 kernels and the host side.
//
// Every function reproduces, bit for bit, one operation of the reference engine
// (dayaswaroopchavali/gemma4-e2b-laptop-cpu, engine/gemma4_engine.cpp = E,
// engine/w4g32_avx2.h = W).  The library is compiled with -ffp-contract=off:
// each FMA below is an explicit fmaf()/fma(), placed exactly where the reference
// has an FMA intrinsic or where GCC contracts a multiply-add in its -O3
// -march=x86-64-v3 build.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define G4V_HD __host__ __device__ __forceinline__

namespace g4v {

G4V_HD float as_f32(uint32_t u) { return __builtin_bit_cast(float, u); }
G4V_HD uint32_t as_u32(float f) { return __builtin_bit_cast(uint32_t, f); }
G4V_HD double as_f64(uint64_t u) { return __builtin_bit_cast(double, u); }
G4V_HD uint64_t as_u64(double d) { return __builtin_bit_cast(uint64_t, d); }

// Component-wise selects of 16-byte vectors.  A conditional expression on the vector types
// themselves is lowered through private memory by this compiler; per-lane component selects
// stay in registers.
G4V_HD float4 keep4(bool ok, float4 v) {
  return make_float4(ok ? v.x : 0.f, ok ? v.y : 0.f, ok ? v.z : 0.f, ok ? v.w : 0.f);
}
G4V_HD uint4 keep4(bool ok, uint4 v) {
  return make_uint4(ok ? v.x : 0u, ok ? v.y : 0u, ok ? v.z : 0u, ok ? v.w : 0u);
}
G4V_HD uint4 sel4(bool c, uint4 a, uint4 b) {
  return make_uint4(c ? a.x : b.x, c ? a.y : b.y, c ? a.z : b.z, c ? a.w : b.w);
}

// W:15 bf16 -> fp32 widening
G4V_HD float bf2f(uint16_t b) { return as_f32((uint32_t)b << 16); }

// E:34 f2bf, round to nearest even (NaN keeps a quiet payload)
G4V_HD uint16_t f2bf(float f) {
  uint32_t u = as_u32(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// E:35 r16 / E:37-42 rbf8: round to bf16 and widen back
G4V_HD float r16(float f) {
  uint32_t u = as_u32(f);
  return as_f32((u + 0x7fffu + ((u >> 16) & 1u)) & 0xFFFF0000u);
}

// E:43-53 exp8 (one lane): Cephes expf (S. L. Moshier) in the engine's FMA order.
G4V_HD float exp8(float x) {
  float a = (x > -87.3f) ? x : -87.3f;  // _mm256_max_ps(x, c): c unless x > c
  x = (a < 88.3f) ? a : 88.3f;          // _mm256_min_ps(a, c): c unless a < c
  float fx = floorf(fmaf(x, 1.44269504088896341f, 0.5f));
  x = fmaf(-fx, 0.693359375f, x);
  x = fmaf(-fx, -2.12194440e-4f, x);
  float z = x * x;
  float y = 1.9875691500E-4f;
  y = fmaf(y, x, 1.3981999507E-3f);
  y = fmaf(y, x, 8.3334519073E-3f);
  y = fmaf(y, x, 4.1665795894E-2f);
  y = fmaf(y, x, 1.6666665459E-1f);
  y = fmaf(y, x, 5.0000001201E-1f);
  y = fmaf(y, z, x + 1.0f);
  int32_t n = ((int32_t)fx + 127) << 23;
  return y * as_f32((uint32_t)n);
}

// E:54-60 gelu8 (one lane): 0.5 x (1 + tanh(u)), tanh(u) = 1 - 2 / (exp8(2u) + 1)
G4V_HD float gelu8(float x) {
  float x3 = (x * x) * x;
  float u = 0.7978845608028654f * fmaf(0.044715f, x3, x);
  float e = exp8(2.0f * u);
  float th = 1.0f - 2.0f / (e + 1.0f);
  return (0.5f * x) * (1.0f + th);
}

// W:41-44 hsum of 8 lanes: ((r0+r4)+(r1+r5))+((r2+r6)+(r3+r7))
G4V_HD float hsum8(const float* r) {
  float a0 = r[0] + r[4], a1 = r[1] + r[5], a2 = r[2] + r[6], a3 = r[3] + r[7];
  return (a0 + a1) + (a2 + a3);
}

// The same sum over the 8 consecutive lanes of a wavefront that each hold one r[j] (lane j of
// the group): a_j = r_j + r_{j^4}, then + lane j^1, then + lane j^2, every lane ending with
// ((r0+r4)+(r1+r5))+((r2+r6)+(r3+r7)).  Data-parallel primitive moves (within rows of 16
// lanes) replace the LDS permute a generic shuffle would use.  (The host pass parses but never
// runs these.)
__device__ __forceinline__ float dpp_f(float v, int ctrl_sel) {
#if defined(__HIP_DEVICE_COMPILE__)
  const int x = __builtin_bit_cast(int, v);
  int y;
  switch (ctrl_sel) {  // constant after inlining
    case 0: y = __builtin_amdgcn_update_dpp(0, x, 0x104, 0xF, 0xF, false); break;  // row_shl:4
    case 1: y = __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, false); break;  // row_shr:4
    case 2: y = __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false); break;   // quad_perm 1,0,3,2
    default: y = __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false); break;  // quad_perm 2,3,0,1
  }
  return __builtin_bit_cast(float, y);
#else
  (void)ctrl_sel;
  return v;
#endif
}
__device__ __forceinline__ float hsum8_lanes(float v) {
  const float up = dpp_f(v, 0), dn = dpp_f(v, 1);
  v = v + ((threadIdx.x & 4) ? dn : up);
  v = v + dpp_f(v, 2);
  return v + dpp_f(v, 3);
}

// libm expf as the reference's host links it (glibc 2.35, FMA code path), used by the split
// merge at E:1028.  Restated from glibc's published table method (sysdeps/ieee754/flt-32/
// e_expf.c, Szabolcs Nagy): N = 32 table entries 2^(i/32), a degree-3 polynomial in double,
// every multiply-add fused.  Arguments here are always <= 0; below -0x1.9fe368p6 the result
// underflows to +0 exactly as glibc returns it.  Checked against the host expf on every
// float in [-inf, 0].
struct ExpfTab {
  uint64_t t[32];
};
G4V_HD float libm_expf_neg(float x, const uint64_t* T) {
  if (x < -0x1.9fe368p6f) return 0.0f;
  const double N = 32.0;
  const double C0 = 0x1.c6af84b912394p-5 / N / N / N, C1 = 0x1.ebfce50fac4f3p-3 / N / N,
               C2 = 0x1.62e42ff0c52d6p-1 / N;
  const double InvLn2N = 0x1.71547652b82fep+0 * N, Shift = 0x1.8p+52;
  double xd = (double)x;
  double kd = fma(InvLn2N, xd, Shift);
  uint64_t ki = as_u64(kd);
  kd -= Shift;
  double r = fma(InvLn2N, xd, -kd);
  uint64_t t = T[ki % 32];
  t += ki << (52 - 5);
  double s = as_f64(t);
  double z = fma(C0, r, C1);
  double r2 = r * r;
  double y = fma(C2, r, 1.0);
  y = fma(z, r2, y);
  y = y * s;
  return (float)y;
}

// asuint64(2^(i/32)) - (i << 47), the correctly rounded doubles of the table method
#define G4V_EXPF_TABLE                                                                        \
  {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
   0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
   0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
   0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
   0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
   0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
   0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
   0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}

// monotone integer key of a float (total order of non-NaN values) for atomic max/min
G4V_HD int32_t fkey(float f) {
  int32_t i = (int32_t)as_u32(f);
  return i >= 0 ? i : (int32_t)(i ^ 0x7fffffff);
}
G4V_HD float fkey_inv(int32_t k) {
  return as_f32((uint32_t)(k >= 0 ? k : (k ^ 0x7fffffff)));
}

// ---- counter-based generator of the synthetic stack (identical formulas on host and device) ----
G4V_HD uint64_t rng_hash(uint64_t seed, uint64_t i) {
  uint64_t z = seed + (i + 1ull) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
G4V_HD float rng_normal(uint64_t seed, uint64_t i) {
  uint64_t a = rng_hash(seed, 2 * i), b = rng_hash(seed, 2 * i + 1);
  int64_t s = 0;
  for (int k = 0; k < 4; ++k) s += (int64_t)((a >> (16 * k)) & 0xFFFF) + (int64_t)((b >> (16 * k)) & 0xFFFF);
  int32_t v = (int32_t)(2 * s - 8 * 65535);
  return (float)v * 0x1.3988e2p-17f;
}
G4V_HD float rng_unif(uint64_t seed, uint64_t i) { return (float)(rng_hash(seed, i) >> 40) * 0x1p-24f; }
G4V_HD uint64_t rng_stream(uint64_t seed, uint64_t tag) {
  return rng_hash(seed * 0x2545F4914F6CDD1Dull + tag, 0x5851F42D4C957F2Dull);
}

}  // namespace g4v
