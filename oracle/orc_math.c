/*
 * orc_math.c -- oracle restatement of the build's decision arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY (see thrml_oracle.h).
 *
 * The reference samples spins with `uniform.lower_equal(sigmoid(2*gamma))`
 * (crates/thrml-samplers/src/spin_gibbs.rs:95-97) and categories with
 * `argmax(theta - log(-log(u)))` (crates/thrml-samplers/src/softmax.rs:86-93).
 * Burn's sigmoid/log rounding is not pinned (its source is not vendored), so
 * the build defines one f32 implementation, written out here a second time,
 * independently of the product header, so that the GPU and this oracle must
 * agree bit for bit:
 *
 *   exp(y):  Cody-Waite reduction y = k ln2 + r, k = rint(y * log2 e), with
 *            ln2 split into the fdlibm e_expf.c pair (0x3f317200, 0x35bfbe8e)
 *            and two fused multiply-adds; exp(r) by its Taylor series to
 *            degree 7 (coefficients 1/n!) in Horner form; times 2^k built
 *            from the exponent field.
 *   sigmoid(x) = 1 / (1 + exp(-x)) with x clamped to [-80, 80] (no
 *            denormals anywhere; the clamp changes no decision because every
 *            p < 2^-24 tests the same as 0 against a 24-bit uniform).
 *   log(x):  x = m 2^e with m in [sqrt(1/2), sqrt(2)), s = (m-1)/(m+1),
 *            log m = 2 atanh s = 2 s (1 + s^2/3 + s^4/5 + s^6/7 + s^8/9),
 *            plus e ln2 (same ln2 split).
 *
 * Every multiply-add is explicit (fmaf) or explicitly unfused; the file is
 * compiled with -ffp-contract=off.
 */
#include <math.h>
#include <string.h>

#include "thrml_oracle.h"

static float bits_to_f(uint32_t b) {
  float f;
  memcpy(&f, &b, 4);
  return f;
}
static uint32_t f_to_bits(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  return b;
}

#define ORC_LOG2E 1.44269502f
#define ORC_LN2_HI 0.693145751953125f     /* 0x3f317200 */
#define ORC_LN2_LO 1.428606765330187e-06f /* 0x35bfbe8e */

float orc_exp(float y) {
  /* y must lie in [-80, 80]; callers clamp. */
  float t = y * ORC_LOG2E;
  float k = rintf(t);
  float r = fmaf(k, -ORC_LN2_HI, y);
  r = fmaf(k, -ORC_LN2_LO, r);
  float p = 1.0f / 5040.0f;
  p = fmaf(p, r, 1.0f / 720.0f);
  p = fmaf(p, r, 1.0f / 120.0f);
  p = fmaf(p, r, 1.0f / 24.0f);
  p = fmaf(p, r, 1.0f / 6.0f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int ki = (int)k;
  float scale = bits_to_f((uint32_t)(ki + 127) << 23);
  return p * scale;
}

float orc_sigmoid(float x) {
  if (x > 80.0f) x = 80.0f;
  if (x < -80.0f) x = -80.0f;
  float e = orc_exp(-x);
  float d = 1.0f + e;
  return 1.0f / d;
}

float orc_log(float x) {
  /* x in (0, 2^64), normal. */
  uint32_t b = f_to_bits(x);
  int e = (int)((b >> 23) & 0xffu) - 127;
  uint32_t mb = (b & 0x007fffffu) | 0x3f800000u; /* m in [1,2) */
  if (mb > 0x3fb504f3u) {                          /* m > sqrt(2) */
    mb -= 0x00800000u;                             /* m /= 2 */
    e += 1;
  }
  float m = bits_to_f(mb);
  float s = (m - 1.0f) / (m + 1.0f);
  float s2 = s * s;
  float q = 1.0f / 9.0f;
  q = fmaf(q, s2, 1.0f / 7.0f);
  q = fmaf(q, s2, 1.0f / 5.0f);
  q = fmaf(q, s2, 1.0f / 3.0f);
  q = fmaf(q, s2, 1.0f);
  float lm = 2.0f * s * q;
  float ef = (float)e;
  float lo = fmaf(ef, ORC_LN2_LO, lm);
  return fmaf(ef, ORC_LN2_HI, lo);
}

float orc_gumbel(uint32_t word) {
  /* u = odd 24-bit integer / 2^24: never 0 or 1 (the reference clips its
   * uniforms to [1e-10, 1-1e-10], softmax.rs:69-73). */
  float u = (float)((word >> 8) | 1u) * 0x1p-24f;
  float l1 = orc_log(u);     /* < 0 */
  float l2 = orc_log(-l1);   /* log(-log u) */
  return -l2;
}

void orc_map_f32(int fn, const float *x, float *y, size_t n) {
  for (size_t i = 0; i < n; i++) {
    switch (fn) {
      case 0: y[i] = orc_exp(x[i]); break;
      case 1: y[i] = orc_sigmoid(x[i]); break;
      default: y[i] = orc_log(x[i]); break;
    }
  }
}

void orc_map_gumbel(const uint32_t *w, float *y, size_t n) {
  for (size_t i = 0; i < n; i++) y[i] = orc_gumbel(w[i]);
}
