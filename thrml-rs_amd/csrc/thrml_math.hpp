// thrml_math.hpp -- the f32 decision arithmetic of the sweep, for host and
// device, rounding step by rounding step identical on both.
//
// The reference samples a spin as `uniform.lower_equal(sigmoid(2*gamma))`
// (crates/thrml-samplers/src/spin_gibbs.rs:95-97) and a category as the first
// argmax of `theta - log(-log(u))` (crates/thrml-samplers/src/softmax.rs:86-93).
// Burn's sigmoid and log are not pinned (not vendored), so this build defines
// them from published methods and uses the same definition on the GPU and in
// the CPU oracle:
//
//   exp(y), y in [-80, 80]: Cody-Waite reduction y = k ln2 + r with
//     k = rint(y * log2(e)) and the two-constant ln2 split of fdlibm's
//     e_expf.c (0x3f317200 + 0x35bfbe8e), applied with fused multiply-adds;
//     exp(r) = Taylor polynomial of degree 7 (1/n! coefficients), Horner form
//     with fused multiply-adds; result times 2^k (exact, normal range only).
//   sigmoid(x) = 1 / (1 + exp(-x)), x first clamped to [-80, 80].  The clamp
//     changes no decision: any p below 2^-24 compares like 0 with a 24-bit
//     uniform, and above 80 the sum 1 + exp(-x) already rounds to 1.
//   log(x), x normal and positive: x = m 2^e with m in [sqrt(1/2), sqrt(2)),
//     s = (m - 1) / (m + 1), log(m) = 2 s (1 + s^2/3 + s^4/5 + s^6/7 + s^8/9)
//     (the atanh series), plus e ln2 with the same split.
//
// Division is IEEE correctly rounded on the host and under hipcc's default
// device lowering; all other steps are explicit.  Every translation unit that
// includes this header is compiled with -ffp-contract=off.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define THRML_MHD __host__ __device__ __forceinline__
#else
#define THRML_MHD inline
#endif

#if !defined(__HIP_DEVICE_COMPILE__)
#include <cmath>
#endif

namespace thrml {

// Division of an index by a launch constant d without a divide: round-up
// reciprocal.  With l = ceil(log2 d) and p = 31 + l, m = ceil(2^p / d) fits
// in 32 bits (d > 2^(l-1)), and floor(x m / 2^p) = floor(x / d) for every
// x < 2^31: x m / 2^p = x / d + x (m d - 2^p) / (d 2^p), and the error term
// is below 2^-l <= 1/d, too small to cross the next multiple of 1/d.  The
// quotient is mulhi(x, m) >> (p - 32) (one scalar multiply-high for a
// wave-uniform x, where a plain '/' would expand into a float-reciprocal
// sequence on the vector unit); m = 0 marks d = 1.
struct FastDiv {
  uint32_t d, m, s;
};
inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f{d, 0u, 0u};
  if (d > 1u) {
    uint32_t l = 0u;
    while ((1ull << l) < d) ++l;
    const uint32_t p = 31u + l;
    f.m = (uint32_t)(((1ull << p) + d - 1ull) / d);
    f.s = p - 32u;
  }
  return f;
}
THRML_MHD uint32_t fdiv(uint32_t x, FastDiv f) {
  return f.m ? (uint32_t)(((uint64_t)x * f.m) >> 32) >> f.s : x;
}

THRML_MHD float f_fma(float a, float b, float c) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_fmaf(a, b, c);
#else
  return std::fma(a, b, c);
#endif
}

THRML_MHD float f_rint(float a) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_rintf(a);
#else
  return std::rint(a);
#endif
}

THRML_MHD float bitsf(uint32_t b) { return __builtin_bit_cast(float, b); }
THRML_MHD uint32_t fbits(float f) { return __builtin_bit_cast(uint32_t, f); }

// exp for y in [-80, 80].
THRML_MHD float exp_b(float y) {
  const float log2e = 1.44269502f;
  const float ln2_hi = bitsf(0x3f317200u);
  const float ln2_lo = bitsf(0x35bfbe8eu);
  float k = f_rint(y * log2e);
  float r = f_fma(k, -ln2_hi, y);
  r = f_fma(k, -ln2_lo, r);
  // Taylor coefficients 1/7!, 1/6!, ..., 1/1!, 1/0!
  float p = f_fma(1.0f / 5040.0f, r, 1.0f / 720.0f);
  p = f_fma(p, r, 1.0f / 120.0f);
  p = f_fma(p, r, 1.0f / 24.0f);
  p = f_fma(p, r, 1.0f / 6.0f);
  p = f_fma(p, r, 0.5f);
  p = f_fma(p, r, 1.0f);
  p = f_fma(p, r, 1.0f);
  const uint32_t e = (uint32_t)((int)k + 127) << 23;
  return p * bitsf(e);
}

THRML_MHD float sigmoid_b(float x) {
  x = x > 80.0f ? 80.0f : x;
  x = x < -80.0f ? -80.0f : x;
  const float den = 1.0f + exp_b(-x);
  return 1.0f / den;
}

// log for positive normal x.
THRML_MHD float log_b(float x) {
  const float ln2_hi = bitsf(0x3f317200u);
  const float ln2_lo = bitsf(0x35bfbe8eu);
  uint32_t b = fbits(x);
  int e = (int)((b >> 23) & 0xffu) - 127;
  uint32_t mb = (b & 0x007fffffu) | 0x3f800000u;
  const bool big = mb > 0x3fb504f3u;  // m > sqrt(2): halve m
  mb = big ? mb - 0x00800000u : mb;
  e = big ? e + 1 : e;
  const float m = bitsf(mb);
  const float s = (m - 1.0f) / (m + 1.0f);
  const float s2 = s * s;
  float q = f_fma(1.0f / 9.0f, s2, 1.0f / 7.0f);
  q = f_fma(q, s2, 1.0f / 5.0f);
  q = f_fma(q, s2, 1.0f / 3.0f);
  q = f_fma(q, s2, 1.0f);
  const float lm = (2.0f * s) * q;
  const float ef = (float)e;
  return f_fma(ef, ln2_hi, f_fma(ef, ln2_lo, lm));
}

// Full-range variants for the kernel-level exports, whose inputs are any
// floats (the sweep kernels only ever pass the ranges above).  On [-80, 80]
// exp_full equals exp_b and sigmoid_full equals sigmoid_b; log_full equals
// log_b on positive normal floats.  Outside, they give the IEEE limits:
// exp_full scales by 2^k in two exact-or-once-rounded steps where 2^k is not
// a normal float (subnormal and near-overflow results), is 0 below -104
// (e^-104 is under half the smallest subnormal) and +inf above 100;
// log_full(+-0) = -inf, log_full(+inf) = +inf, NaN for negative or NaN input,
// and subnormal x = m 2^e is reduced with its true exponent.
THRML_MHD float exp_full(float y) {
  if (!(y == y)) return y;
  if (y > 100.0f) return bitsf(0x7f800000u);
  if (y < -104.0f) return 0.0f;
  const float log2e = 1.44269502f;
  const float ln2_hi = bitsf(0x3f317200u);
  const float ln2_lo = bitsf(0x35bfbe8eu);
  float k = f_rint(y * log2e);
  float r = f_fma(k, -ln2_hi, y);
  r = f_fma(k, -ln2_lo, r);
  float p = f_fma(1.0f / 5040.0f, r, 1.0f / 720.0f);
  p = f_fma(p, r, 1.0f / 120.0f);
  p = f_fma(p, r, 1.0f / 24.0f);
  p = f_fma(p, r, 1.0f / 6.0f);
  p = f_fma(p, r, 0.5f);
  p = f_fma(p, r, 1.0f);
  p = f_fma(p, r, 1.0f);
  const int ki = (int)k;
  if (ki > 127) return (p * bitsf((uint32_t)(ki - 64 + 127) << 23)) * 0x1p64f;
  if (ki < -126) return (p * bitsf((uint32_t)(ki + 64 + 127) << 23)) * 0x1p-64f;
  return p * bitsf((uint32_t)(ki + 127) << 23);
}

THRML_MHD float sigmoid_full(float x) { return 1.0f / (1.0f + exp_full(-x)); }

THRML_MHD float log_full(float x) {
  if (!(x == x)) return x;
  if (x < 0.0f) return bitsf(0x7fc00000u);
  if (x == 0.0f) return bitsf(0xff800000u);
  const uint32_t b = fbits(x);
  if (b == 0x7f800000u) return x;
  int e;
  uint32_t mb;
  if ((b >> 23) == 0u) {  // subnormal: b 2^-149, top bit of b below bit 23
    const int lz = __builtin_clz(b) - 8;
    mb = ((b << lz) & 0x007fffffu) | 0x3f800000u;
    e = -126 - lz;
  } else {
    e = (int)((b >> 23) & 0xffu) - 127;
    mb = (b & 0x007fffffu) | 0x3f800000u;
  }
  const float ln2_hi = bitsf(0x3f317200u);
  const float ln2_lo = bitsf(0x35bfbe8eu);
  const bool big = mb > 0x3fb504f3u;
  mb = big ? mb - 0x00800000u : mb;
  e = big ? e + 1 : e;
  const float m = bitsf(mb);
  const float s = (m - 1.0f) / (m + 1.0f);
  const float s2 = s * s;
  float q = f_fma(1.0f / 9.0f, s2, 1.0f / 7.0f);
  q = f_fma(q, s2, 1.0f / 5.0f);
  q = f_fma(q, s2, 1.0f / 3.0f);
  q = f_fma(q, s2, 1.0f);
  const float lm = (2.0f * s) * q;
  const float ef = (float)e;
  return f_fma(ef, ln2_hi, f_fma(ef, ln2_lo, lm));
}

// Uniform in (0,1) for the Gumbel draw: odd 24-bit integer over 2^24.
THRML_MHD float gumbel_uniform(uint32_t w) { return (float)((w >> 8) | 1u) * 0x1p-24f; }

// -log(-log(u)) of a keystream word.
THRML_MHD float gumbel_b(uint32_t w) {
  const float l1 = log_b(gumbel_uniform(w));
  return -log_b(-l1);
}

// Uniform in [0,1) for spin updates: 24-bit integer over 2^24.
THRML_MHD float spin_uniform(uint32_t w) { return (float)(w >> 8) * 0x1p-24f; }

// Keystream-word threshold of a Bernoulli(p) draw: for every word w,
//   (spin_uniform(w) <= p)  <=>  (w <= word_threshold(p)).
// spin_uniform(w) <= p  <=>  (w >> 8) <= floor(p * 2^24)  (p * 2^24 is exact).
THRML_MHD uint32_t word_threshold(float p) {
  if (!(p < 1.0f)) return 0xffffffffu;
  const uint32_t m = (uint32_t)(p * 16777216.0f);
  return (m << 8) | 0xffu;
}

}  // namespace thrml
