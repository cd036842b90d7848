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
#include <stdio.h>
#include <stdlib.h>
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

/* Full-range forms (kernel-level exports, any float input).  On [-80, 80]
 * orc_exp_full is orc_exp; orc_log_full is orc_log on positive normals.
 * Elsewhere the IEEE limits: exp is 0 below -104 (e^-104 is under half the
 * smallest subnormal) and +inf above 100, and
 * 2^k that is not a normal float is applied as 2^(k -+ 64) then 2^(+-64)
 * (the first product exact, the second rounding once); log(+-0) = -inf,
 * log(+inf) = +inf, NaN for negative or NaN x, subnormal x = m 2^e with
 * its true exponent. */
float orc_exp_full(float y) {
  if (isnan(y)) return y;
  if (y > 100.0f) return INFINITY;
  if (y < -104.0f) return 0.0f;
  float k = rintf(y * ORC_LOG2E);
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
  if (ki > 127) return (p * bits_to_f((uint32_t)(ki - 64 + 127) << 23)) * 0x1p64f;
  if (ki < -126) return (p * bits_to_f((uint32_t)(ki + 64 + 127) << 23)) * 0x1p-64f;
  return p * bits_to_f((uint32_t)(ki + 127) << 23);
}

float orc_sigmoid_full(float x) {
  float e = orc_exp_full(-x);
  float d = 1.0f + e;
  return 1.0f / d;
}

float orc_log_full(float x) {
  if (isnan(x)) return x;
  if (x < 0.0f) return NAN;
  if (x == 0.0f) return -INFINITY;
  if (isinf(x)) return x;
  uint32_t b = f_to_bits(x);
  int e;
  uint32_t mb;
  if ((b >> 23) == 0u) {
    /* subnormal: normalise the 23-bit fraction */
    int lz = 0;
    while (!((b << lz) & 0x00800000u)) lz++;
    mb = ((b << lz) & 0x007fffffu) | 0x3f800000u;
    e = -126 - lz;
  } else {
    e = (int)((b >> 23) & 0xffu) - 127;
    mb = (b & 0x007fffffu) | 0x3f800000u;
  }
  if (mb > 0x3fb504f3u) {
    mb -= 0x00800000u;
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

/* The reference's FusedKernelBackend kernels restated
 * (crates/thrml-kernels/src/gumbel_argmax/kernel.rs:47-88,
 * crates/thrml-kernels/src/sigmoid_bernoulli/kernel.rs:34-55): gumbel =
 * 0 - log(0 - log(u)), perturbed = logit + gumbel, index of the first
 * maximum under '>' (a NaN score is never taken after index 0);
 * sample = (u < 1 / (1 + exp(0 - 2 gamma))). */
void orc_gumbel_argmax(const float *logits, const float *u, int32_t *out, size_t n, uint32_t q) {
  for (size_t r = 0; r < n; r++) {
    const float *l = logits + r * q, *ur = u + r * q;
    float best = l[0] + (0.0f - orc_log_full(0.0f - orc_log_full(ur[0])));
    int32_t arg = 0;
    for (uint32_t k = 1; k < q; k++) {
      float v = l[k] + (0.0f - orc_log_full(0.0f - orc_log_full(ur[k])));
      if (v > best) {
        best = v;
        arg = (int32_t)k;
      }
    }
    out[r] = arg;
  }
}

void orc_sigmoid_bernoulli(const float *gamma, const float *u, float *out, size_t n) {
  for (size_t i = 0; i < n; i++) {
    float two_g = 2.0f * gamma[i];
    float prob = 1.0f / (1.0f + orc_exp_full(0.0f - two_g));
    out[i] = u[i] < prob ? 1.0f : 0.0f;
  }
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
      case 3: y[i] = orc_exp_full(x[i]); break;
      case 4: y[i] = orc_sigmoid_full(x[i]); break;
      case 5: y[i] = orc_log_full(x[i]); break;
      default: y[i] = orc_log(x[i]); break;
    }
  }
}

void orc_map_gumbel(const uint32_t *w, float *y, size_t n) {
  for (size_t i = 0; i < n; i++) y[i] = orc_gumbel(w[i]);
}

/* Superblock offsets over the free blocks (BlockGibbsSpec::new,
 * crates/thrml-samplers/src/program.rs:28-64 flattens Vec<SuperBlock> into
 * free_blocks and keeps one index group per superblock).  n_sb = 0 gives one
 * superblock per free block. */
uint32_t *orc_sb_partition(uint32_t n_free, uint32_t n_sb, const uint32_t *off,
                           uint32_t *n_out, char *err, size_t errlen) {
  if (n_sb == 0) {
    uint32_t *r = (uint32_t *)malloc(((size_t)n_free + 1) * sizeof(uint32_t));
    for (uint32_t b = 0; b <= n_free; b++) r[b] = b;
    *n_out = n_free;
    return r;
  }
  if (!off || off[0] != 0 || off[n_sb] != n_free) {
    if (err && errlen)
      snprintf(err, errlen, "superblock offsets must start at 0 and end at the number of free blocks");
    return NULL;
  }
  for (uint32_t s = 0; s < n_sb; s++)
    if (off[s + 1] < off[s]) {
      if (err && errlen) snprintf(err, errlen, "superblock offsets must not decrease");
      return NULL;
    }
  uint32_t *r = (uint32_t *)malloc(((size_t)n_sb + 1) * sizeof(uint32_t));
  memcpy(r, off, ((size_t)n_sb + 1) * sizeof(uint32_t));
  *n_out = n_sb;
  return r;
}

/* batch_gather_fused (crates/thrml-kernels/src/batch_gather/kernel.rs:1-30,
 * launched by batch_gather/forward.rs): out[b] = weights[lin] with lin =
 * b * batch_stride + sum_i (u32)indices[b * n + i] * strides[i] in wrapping
 * u32 arithmetic; lin >= n_weights gives 0.0 (this build's choice for a read
 * the reference leaves to its backend's bounds checks). */
void orc_batch_gather(const float *w, uint64_t n_w, const int32_t *idx, uint64_t batch,
                      uint32_t n, const uint32_t *strides, uint32_t batch_stride, float *out) {
  for (uint64_t b = 0; b < batch; b++) {
    uint32_t lin = (uint32_t)b * batch_stride;
    for (uint32_t i = 0; i < n; i++) lin += (uint32_t)idx[b * n + i] * strides[i];
    out[b] = lin < n_w ? w[lin] : 0.0f;
  }
}
