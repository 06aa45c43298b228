/* g4_rng.h -- counter-based integer generator for the synthetic inputs.
 *
 * TEST INFRASTRUCTURE (oracle/): used by the oracle, the reference harness
 * and the tests to build identical seeded inputs.  Nothing in the product
 * links it.
 *
 * Every value is a pure function of (seed, index), built from integer
 * arithmetic and exactly one IEEE fp32 rounding, so numpy, C and HIP produce
 * identical bits without any libm dependence:
 *   h(seed, i)   = splitmix64 finaliser of seed + (i + 1) * 0x9E3779B97F4A7C15
 *   normal(s, i) = sum of eight 16-bit lanes of h(s, 2i) and h(s, 2i+1),
 *                  centred and scaled to unit variance (Irwin-Hall, 8 terms,
 *                  tails bounded at +-4.9 sigma)
 *   unif(s, i)   = (h >> 40) * 2^-24 in [0, 1)
 */
#ifndef G4_RNG_H
#define G4_RNG_H
#include <stdint.h>

static inline uint64_t g4r_hash(uint64_t seed, uint64_t i) {
  uint64_t z = seed + (i + 1ull) * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

/* 1 / (2 * 65536 * sqrt(8/12)) rounded to fp32: the centred 8-lane sum
 * 2*s - 8*65535 has standard deviation 2*65536*sqrt(8/12) ~= 107019.84 */
#define G4R_NORM_SCALE 0x1.3988e2p-17f

static inline float g4r_normal(uint64_t seed, uint64_t i) {
  uint64_t a = g4r_hash(seed, 2 * i), b = g4r_hash(seed, 2 * i + 1);
  int64_t s = 0;
  for (int k = 0; k < 4; ++k) s += (int64_t)((a >> (16 * k)) & 0xFFFF) + (int64_t)((b >> (16 * k)) & 0xFFFF);
  int32_t v = (int32_t)(2 * s - 8 * 65535);
  return (float)v * G4R_NORM_SCALE;
}

static inline float g4r_unif(uint64_t seed, uint64_t i) {
  return (float)(g4r_hash(seed, i) >> 40) * 0x1p-24f;
}

/* integer uniform on [lo, hi] */
static inline int32_t g4r_int(uint64_t seed, uint64_t i, int32_t lo, int32_t hi) {
  return lo + (int32_t)(g4r_hash(seed, i) % (uint64_t)(hi - lo + 1));
}

/* stream seed for tensor `tag` of a run with base seed `seed` */
static inline uint64_t g4r_stream(uint64_t seed, uint64_t tag) {
  return g4r_hash(seed * 0x2545F4914F6CDD1Dull + tag, 0x5851F42D4C957F2Dull);
}
#endif
