// synth.h -- deterministic synthetic-data generator shared by host and device.
//
// The same element index gives the same bits on the CPU (g++) and on gfx950
// (hipcc): every step is integer arithmetic or an IEEE-754 double +, -, *, /
// with contraction disabled, so no libm routine (whose last bits differ
// between glibc and the device math library) is involved.
//
//   u64  h  = splitmix64(key + i * golden)            (Steele, Lea, Flood 2014)
//   u1  = (h >> 32 + 1) / 2^32 in (0, 1],  u2 = (h & 0xFFFFFFFF) / 2^32 in [0, 1)
//   z   = sqrt(-2 ln u1) * cos(2 pi u2)               (Box-Muller, cosine branch)
//   ln  : exponent split + atanh series, sqrt : Newton, cos : quadrant + Taylor
//   out = (float)(mean + std * z), optionally rounded to bf16 (RNE)
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define GH_HD __host__ __device__ inline
#else
#define GH_HD static inline
#endif

// Contraction (a*b+c -> fma) would change the last bits on one side only.
#if defined(__clang__)
#define GH_NOCONTRACT _Pragma("clang fp contract(off)")
#else
#define GH_NOCONTRACT
#endif

GH_HD uint64_t gh_splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

GH_HD double gh_u64_as_f64(uint64_t b) {
  double d;
  __builtin_memcpy(&d, &b, 8);
  return d;
}

GH_HD uint64_t gh_f64_bits(double d) {
  uint64_t b;
  __builtin_memcpy(&b, &d, 8);
  return b;
}

// Natural log of a positive normal double.
GH_HD double gh_det_log(double x) {
  GH_NOCONTRACT
  uint64_t b = gh_f64_bits(x);
  int e = (int)((b >> 52) & 0x7FF) - 1023;
  double m = gh_u64_as_f64((b & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull);
  if (m > 1.4142135623730951) {
    m = m * 0.5;
    e += 1;
  }
  double f = (m - 1.0) / (m + 1.0);
  double s = f * f;
  double p = 1.0 / 25.0;
  p = p * s + 1.0 / 23.0;
  p = p * s + 1.0 / 21.0;
  p = p * s + 1.0 / 19.0;
  p = p * s + 1.0 / 17.0;
  p = p * s + 1.0 / 15.0;
  p = p * s + 1.0 / 13.0;
  p = p * s + 1.0 / 11.0;
  p = p * s + 1.0 / 9.0;
  p = p * s + 1.0 / 7.0;
  p = p * s + 1.0 / 5.0;
  p = p * s + 1.0 / 3.0;
  p = p * s + 1.0;
  return (double)e * 0.69314718055994530942 + 2.0 * f * p;
}

// Square root of a non-negative double by Newton's iteration.
GH_HD double gh_det_sqrt(double a) {
  GH_NOCONTRACT
  if (!(a > 0.0)) return 0.0;
  double y = gh_u64_as_f64((gh_f64_bits(a) >> 1) + 0x1FF8000000000000ull);
  for (int i = 0; i < 6; i++) y = 0.5 * (y + a / y);
  return y;
}

// cos(2 pi j / 2^32).
GH_HD double gh_det_cos_turn(uint32_t j) {
  GH_NOCONTRACT
  uint32_t quad = j >> 30;
  double t = (double)(j & 0x3FFFFFFFu) * (1.0 / 4294967296.0);  // [0, 1/4) turn
  double a = t * 6.28318530717958647692;
  double a2 = a * a;
  double c = 1.0 / 20922789888000.0;          // 1/16!
  c = c * (-a2) + 1.0 / 87178291200.0;        // 1/14!
  c = c * (-a2) + 1.0 / 479001600.0;          // 1/12!
  c = c * (-a2) + 1.0 / 3628800.0;            // 1/10!
  c = c * (-a2) + 1.0 / 40320.0;              // 1/8!
  c = c * (-a2) + 1.0 / 720.0;
  c = c * (-a2) + 1.0 / 24.0;
  c = c * (-a2) + 1.0 / 2.0;
  c = c * (-a2) + 1.0;                        // cos a
  double s = 1.0 / 355687428096000.0;         // 1/17!
  s = s * (-a2) + 1.0 / 1307674368000.0;      // 1/15!
  s = s * (-a2) + 1.0 / 6227020800.0;         // 1/13!
  s = s * (-a2) + 1.0 / 39916800.0;           // 1/11!
  s = s * (-a2) + 1.0 / 362880.0;             // 1/9!
  s = s * (-a2) + 1.0 / 5040.0;
  s = s * (-a2) + 1.0 / 120.0;
  s = s * (-a2) + 1.0 / 6.0;
  s = s * (-a2) + 1.0;
  s = s * a;                                  // sin a
  if (quad == 0) return c;
  if (quad == 1) return -s;
  if (quad == 2) return -c;
  return s;
}

GH_HD uint64_t gh_stream_key(uint64_t seed, uint64_t stream) {
  return gh_splitmix64(seed ^ gh_splitmix64(stream ^ 0x5EED5EED5EED5EEDull));
}

// Standard normal draw number i of the (seed, stream) sequence.
GH_HD double gh_normal(uint64_t key, uint64_t i) {
  GH_NOCONTRACT
  uint64_t h = gh_splitmix64(key + i * 0x9E3779B97F4A7C15ull);
  double u1 = ((double)(h >> 32) + 1.0) * (1.0 / 4294967296.0);
  double r = gh_det_sqrt(-2.0 * gh_det_log(u1));
  return r * gh_det_cos_turn((uint32_t)(h & 0xFFFFFFFFu));
}

GH_HD float gh_normal_f32(uint64_t key, uint64_t i, double mean, double stddev) {
  GH_NOCONTRACT
  return (float)(mean + stddev * gh_normal(key, i));
}

// src/tensor.zig:7-13 rounding: bits + 0x7FFF + ((bits >> 16) & 1), then >> 16.
GH_HD uint16_t gh_bf16_rne(float v) {
  uint32_t b;
  __builtin_memcpy(&b, &v, 4);
  return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

// Uniform integer in [0, n) for draw i (used for synthetic token ids).
GH_HD uint32_t gh_uniform_u32(uint64_t key, uint64_t i, uint32_t n) {
  return (uint32_t)(gh_splitmix64(key + i * 0x9E3779B97F4A7C15ull) % (uint64_t)n);
}
