// dev_util.hpp -- device helpers shared by the sweep kernels (gfx950).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "thrml_math.hpp"
#include "thrml_rng.hpp"

namespace thrml {

// Workgroups are dispatched round-robin over the 8 XCDs; remap the launch
// index so that each XCD walks a contiguous range of work (neighbouring rows
// or tiles then share that XCD's L2).
__device__ __forceinline__ uint32_t xcd_remap(uint32_t bid, uint32_t nwg) {
  const uint32_t nx = 8;
  const uint32_t xcd = bid % nx, idx = bid / nx;
  const uint32_t per = nwg / nx, rem = nwg % nx;
  return xcd * per + (xcd < rem ? xcd : rem) + idx;
}

// The raw key words (x[0..7]) of chain `chain` from a [chains][KEY_WORDS]
// table, for kernels whose memory pipeline is busier than their VALU.
__device__ __forceinline__ void load_key8(const uint32_t *__restrict__ keys, uint32_t chain,
                                          uint32_t k[8]) {
  const uint4 *k4 = reinterpret_cast<const uint4 *>(keys + (size_t)chain * KEY_WORDS);
  const uint4 a = k4[0], b = k4[1];
  k[0] = a.x; k[1] = a.y; k[2] = a.z; k[3] = a.w;
  k[4] = b.x; k[5] = b.y; k[6] = b.z; k[7] = b.w;
}

// Stream key of chain `chain` from a [chains][KEY_WORDS] table of expanded
// keys (key_expand), six 16-byte loads.
__device__ __forceinline__ void load_keyx(const uint32_t *__restrict__ keys, uint32_t chain,
                                          uint32_t x[KEY_WORDS]) {
  const uint4 *k4 = reinterpret_cast<const uint4 *>(keys + (size_t)chain * KEY_WORDS);
#pragma unroll
  for (int q = 0; q < KEY_WORDS / 4; ++q) {
    const uint4 v = k4[q];
    x[4 * q] = v.x; x[4 * q + 1] = v.y; x[4 * q + 2] = v.z; x[4 * q + 3] = v.w;
  }
}

// This lane's bit of a wave-uniform 64-bit lane mask.
__device__ __forceinline__ bool lane_bit(uint64_t w) {
  return __builtin_amdgcn_inverse_ballot_w64(w);
}

// v_writelane_b32: lane `L` of `old` takes the wave-uniform `val`.  The lane
// is an immediate (no lane-select hazard).  `val` may be VCC just written by
// a VALU compare (a ballot); reading it back as an explicit SGPR operand needs
// a wait state, which the compiler's hazard pass does not add inside inline
// assembly, hence the s_nop.
template <int L>
__device__ __forceinline__ uint32_t writelane(uint32_t old, uint32_t val) {
  asm("s_nop 1\n\tv_writelane_b32 %0, %1, %2" : "+v"(old) : "s"(__builtin_amdgcn_readfirstlane(val)), "i"(L));
  return old;
}

template <int K, class F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (K > 0) {
    static_for<K - 1>(f);
    f(std::integral_constant<int, K - 1>{});
  }
}

__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  // hides a wave-uniform value from the optimiser, so that loads indexed by
  // it are issued again instead of being kept live across other work
  asm("" : "+s"(v));
  return v;
}

// The spin decision spin_uniform(w) <= sigmoid_b(2 g) of the reference rule
// u <= sigmoid(2 gamma) (crates/thrml-samplers/src/spin_gibbs.rs:95-97) for
// gamma = g, equal to it for every (g, w).  With x = 2g,
//   u <= sigma(x)  <=>  u (1 + e^-x) <= 1,
// and q = fma(u, E, u) with E = 2^(-x log2 e) from the hardware exponential
// is u (1 + e^-x)(1 + t), |t| <= eps_E + 2^-24 (eps_E the largest relative
// error of E against e^-x), while sigmoid_b(x) = sigma(x)(1 + s), |s| <=
// eps_s.  So q <= 1 - SPIN_BAND implies u <= sigmoid_b(x) and q > 1 + SPIN_BAND
// implies u > sigmoid_b(x) whenever SPIN_BAND > eps_E + eps_s + 2^-23:
// thrml_fast_math_check measures eps_E and eps_s over every float g in
// [-40, 40] and the tests require that.  Only q inside the band (probability
// about 3e-5) takes the exact sigmoid_b.  One transcendental per decision.
//
// The product is formed as q 2^24 = fma(v, E, v) with v = w >> 8 = u 2^24
// (exact, and scaling by a power of two commutes with the rounding), against
// thresholds scaled alike.  g is not clamped on this path: for g > 40, E is
// below e^-80 and q rounds to u (the band decides u near 1); for g < -40, q
// exceeds 1 + SPIN_BAND for every u > 0 (E = +inf included), and u = 0 makes
// q NaN, which fails both compares and takes the exact rule.  The exact rule
// clamps g to [-40, 40], which changes no decision: sigmoid_b is 1 above
// x = 80, and below x = -80 it is under 2^-24, the smallest nonzero uniform.
constexpr float SPIN_BAND = 0x1p-16f;

__device__ __forceinline__ float spin_exp_neg(float g) {  // e^(-2g)
  return __builtin_amdgcn_exp2f(g * (-2.0f * 1.44269504f));
}

__device__ __forceinline__ bool spin_decision(float g, uint32_t w) {
  const float v = (float)(w >> 8);
  const float q = __builtin_fmaf(v, spin_exp_neg(g), v);
  bool up = q <= (1.0f - SPIN_BAND) * 0x1p24f;
  const bool band = !(up || q > (1.0f + SPIN_BAND) * 0x1p24f);
  if (band) {
    g = g > 40.0f ? 40.0f : g;
    g = g < -40.0f ? -40.0f : g;
    up = spin_uniform(w) <= sigmoid_b(g * 2.0f);
  }
  return up;
}

// spin_decision for every active lane of the wave, as the mask of lanes that
// take spin up.  The band test is a wave-uniform branch on the mask of lanes
// that neither fast compare decides.
__device__ __forceinline__ uint64_t spin_decision_mask(float g, uint32_t w) {
  const float v = (float)(w >> 8);
  const float q = __builtin_fmaf(v, spin_exp_neg(g), v);
  uint64_t up = __builtin_amdgcn_ballot_w64(q <= (1.0f - SPIN_BAND) * 0x1p24f);
  const uint64_t dn = __builtin_amdgcn_ballot_w64(q > (1.0f + SPIN_BAND) * 0x1p24f);
  const uint64_t band = ~(up | dn) & __builtin_amdgcn_read_exec();
  if (band) {
    g = g > 40.0f ? 40.0f : g;
    g = g < -40.0f ? -40.0f : g;
    up |= __builtin_amdgcn_ballot_w64(lane_bit(band) && spin_uniform(w) <= sigmoid_b(g * 2.0f));
  }
  return up;
}

// 2 acc + (this lane's bit of mask), one v_addc_co_u32 with the mask as the
// carry-in: shifts one lane-selected bit into a per-lane word, high bit first.
// The mask may have been written by a VALU compare just before; reading it as
// the carry-in SGPR operand needs wait states that the hazard pass does not
// add inside inline assembly, hence the s_nop.
__device__ __forceinline__ uint32_t shift_in(uint32_t acc, uint64_t mask) {
  uint32_t d;
  uint64_t co;
  asm("s_nop 1\n\tv_addc_co_u32_e64 %0, %1, %2, %2, %3" : "=v"(d), "=s"(co) : "v"(acc), "s"(mask));
  return d;
}

// Gumbel score of a keystream word from the hardware logarithm (v_log_f32):
// -ln(-ln u) with u = gumbel_uniform(w).  u takes 2^23 values, and over all
// of them |gumbel_fast(w) - gumbel_b(w)| <= 1.91e-6 (measured exhaustively by
// thrml_fast_math_check; the tests require GUMBEL_FAST_ERR).  A categorical
// draw keeps the fast argmax when its top two scores are further apart than
// gumbel_margin, which then makes it equal to the exact argmax; otherwise
// the site is drawn again with gumbel_b.
constexpr float GUMBEL_FAST_ERR = 4e-6f;

// -ln(-ln u) = -ln(ln 2) - ln 2 * log2(-log2 u): two hardware logarithms and
// one fma after the uniform.
__device__ __forceinline__ float gumbel_fast(uint32_t w) {
  const float l = __builtin_amdgcn_logf(gumbel_uniform(w));  // log2 u < 0
  return __builtin_fmaf(__builtin_amdgcn_logf(-l), -0.693147182f, 0.366512921f);
}

// fl(theta + g) and fl(theta + gumbel_fast) differ by at most
// GUMBEL_FAST_ERR + ulp(v) <= GUMBEL_FAST_ERR + |v| 2^-23 for each score v,
// so a gap above twice that (with the ulp bound doubled) fixes the argmax.
__device__ __forceinline__ float gumbel_margin(float best, float second) {
  return 2.0f * GUMBEL_FAST_ERR + (fabsf(best) + fabsf(second)) * 0x1p-22f;
}

// The category of lane-local site s from its theta: fast Gumbel scores and
// the first maximum; if the top two are within gumbel_margin, the exact
// scores (gumbel_b) decide.  blk / have stream the lane's keystream blocks
// (site s, category q takes word OFF + s*Q + q relative to block ctr0).
template <int Q, int OFF = 0>
__device__ __forceinline__ uint32_t potts_pick(const float (&th)[Q], int s, const uint32_t (&key)[8],
                                               uint64_t ctr0, uint32_t (&blk)[16], int &have) {
  float best = 0.0f, second = -INFINITY;
  uint32_t arg = 0;
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const int rel = OFF + s * Q + q;
    if ((rel >> 4) != have) {
      chacha_block<8>(key, ctr0 + (uint64_t)(rel >> 4), blk);
      have = rel >> 4;
    }
    const float v = th[q] + gumbel_fast(blk[rel & 15]);
    if (q == 0) {
      best = v;
    } else if (v > best) {
      second = best;
      best = v;
      arg = (uint32_t)q;
    } else if (v > second) {
      second = v;
    }
  }
  if (!(best - second > gumbel_margin(best, second))) {
    uint32_t eb[16];
    int have2 = -1;
    best = 0.0f;
    arg = 0;
    for (int q = 0; q < Q; ++q) {
      const int rel = OFF + s * Q + q;
      if ((rel >> 4) != have2) {
        chacha_block<8>(key, ctr0 + (uint64_t)(rel >> 4), eb);
        have2 = rel >> 4;
      }
      uint32_t wq = eb[0];
#pragma unroll
      for (int t = 1; t < 16; ++t) wq = ((rel & 15) == t) ? eb[t] : wq;
      const float v = th[q] + gumbel_b(wq);
      if (q == 0 || v > best) {
        best = v;
        arg = (uint32_t)q;
      }
    }
  }
  return arg;
}

// Q contiguous floats at row (16-byte aligned when Q is a multiple of 4:
// rows of q floats in arrays whose rows start at multiples of 4 floats).
template <int Q>
__device__ __forceinline__ void load_row(const float *row, float (&v)[Q]) {
  if constexpr (Q % 4 == 0) {
#pragma unroll
    for (int t = 0; t < Q / 4; ++t) {
      const float4 f = reinterpret_cast<const float4 *>(row)[t];
      v[4 * t] = f.x;
      v[4 * t + 1] = f.y;
      v[4 * t + 2] = f.z;
      v[4 * t + 3] = f.w;
    }
  } else {
#pragma unroll
    for (int q = 0; q < Q; ++q) v[q] = row[q];
  }
}

// Load the 16 floats row[q0 .. q0 + 15] of a row of Q floats (entries
// outside the row are never used, and are loaded from inside it).  AL = 16:
// q0 is a multiple of 16 with q0 + 16 <= Q and row 16-byte aligned (four
// 16-byte loads).  AL = 4: Q and q0 multiples of 4 and row 16-byte aligned,
// so each group of 4 categories lies wholly inside or wholly outside the row;
// a group's start is clamped into 0..Q-4 (four 16-byte loads).  AL = 2 alike
// with Q even and groups of 2 (eight 8-byte loads).  AL = 1: each index
// clamped into 0..Q-1.
template <int AL>
__device__ __forceinline__ void load_chunk16(const float *row, int32_t q0, uint32_t Q,
                                             float (&v)[16]) {
  if constexpr (AL == 16 || AL == 4) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      int32_t q = q0 + 4 * t;
      if constexpr (AL == 4) q = q < 0 ? 0 : q > (int32_t)Q - 4 ? (int32_t)Q - 4 : q;
      const float4 f = *reinterpret_cast<const float4 *>(row + q);
      v[4 * t] = f.x;
      v[4 * t + 1] = f.y;
      v[4 * t + 2] = f.z;
      v[4 * t + 3] = f.w;
    }
  } else if constexpr (AL == 2) {
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      int32_t q = q0 + 2 * t;
      q = q < 0 ? 0 : q > (int32_t)Q - 2 ? (int32_t)Q - 2 : q;
      const float2 f = *reinterpret_cast<const float2 *>(row + q);
      v[2 * t] = f.x;
      v[2 * t + 1] = f.y;
    }
  } else {
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const int32_t q = q0 + t;
      v[t] = row[q < 0 ? 0 : q >= (int32_t)Q ? (int32_t)Q - 1 : q];
    }
  }
}

// The category of a site with Q > 16 categories whose keystream words are
// w0 .. w0 + Q - 1 of the lane's stream (category c: word w0 + c).  The words
// are taken one ChaCha8 block at a time: block k of the site holds categories
// 16k - o .. 16k - o + 15 (o = w0 mod 16; those outside 0..Q-1 are skipped),
// and theta_chunk(k, q0, th) writes th[t] = theta of category q0 + t with
// q0 = 16k - o (entries outside 0..Q-1 are ignored).  Fast Gumbel scores and
// the first maximum, scanned in category order; when the top two are within
// gumbel_margin, theta and the exact scores (gumbel_b) are computed again.
template <typename F>
__device__ __forceinline__ uint32_t wide_pick(uint32_t Q, uint64_t w0, const uint32_t (&key)[8],
                                              F &&theta_chunk) {
  const int32_t o = (int32_t)(w0 & 15u);
  const uint64_t b0 = w0 >> 4;
  const uint32_t nb = ((uint32_t)o + Q + 15u) >> 4;
  float best = -INFINITY, second = -INFINITY;
  uint32_t arg = 0;
  for (uint32_t k = 0; k < nb; ++k) {
    const int32_t q0 = 16 * (int32_t)k - o;
    float th[16];
    theta_chunk(k, q0, th);
    uint32_t blk[16];
    chacha_block<8>(key, b0 + k, blk);
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      // a skipped category scores -inf: it changes neither the maximum nor
      // the runner-up (best >= second throughout)
      const int32_t q = q0 + t;
      const float v = (q >= 0 && q < (int32_t)Q) ? th[t] + gumbel_fast(blk[t]) : -INFINITY;
      const bool gt = v > best;
      second = __builtin_amdgcn_fmed3f(v, best, second);
      arg = gt ? (uint32_t)q : arg;
      best = gt ? v : best;
    }
  }
  if (!(best - second > gumbel_margin(best, second))) {
    best = -INFINITY;
    arg = 0;
    for (uint32_t k = 0; k < nb; ++k) {
      const int32_t q0 = 16 * (int32_t)k - o;
      float th[16];
      theta_chunk(k, q0, th);
      uint32_t blk[16];
      chacha_block<8>(key, b0 + k, blk);
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const int32_t q = q0 + t;
        if (q >= 0 && q < (int32_t)Q) {
          const float v = th[t] + gumbel_b(blk[t]);
          if (q == 0 || v > best) {
            best = v;
            arg = (uint32_t)q;
          }
        }
      }
    }
  }
  return arg;
}

// Top two scores and the category of the first maximum, merged across lanes
// that hold disjoint categories: best and second are the largest and
// second-largest of the union (order-independent for values that are not
// NaN), and on equal bests the lower category wins.
__device__ __forceinline__ void top2_merge(float &best, float &second, uint32_t &arg, float ob,
                                           float os, uint32_t oa) {
  const bool take = ob > best || (ob == best && oa < arg);
  second = fmaxf(fminf(best, ob), fmaxf(second, os));
  arg = take ? oa : arg;
  best = fmaxf(best, ob);
}

// wide_pick with the site's keystream blocks split over the 64 lanes of a
// wave (every lane calls it with the same arguments but its lane index): lane
// l takes blocks l, l + 64, ... (block k holds categories 16k - o ..
// 16k - o + 15, as in wide_pick), keeps the top two fast scores and the first
// maximum of its categories, and a butterfly over the wave merges them; if
// the top two are within gumbel_margin, every lane scores its categories
// again with gumbel_b and the first maximum is merged the same way.  The
// result equals wide_pick's sequential scan: with no NaN the maximum, the
// runner-up and the first index of the maximum do not depend on the order of
// the merges; a NaN score (a NaN or infinite weight) sends the item to
// wide_pick itself, which every lane then runs alike.  Returns the category
// in every lane.
template <typename F>
__device__ __forceinline__ uint32_t wave_pick(uint32_t Q, uint64_t w0, const uint32_t (&key)[8],
                                              uint32_t lane, F &&theta_chunk) {
  const int32_t o = (int32_t)(w0 & 15u);
  const uint64_t b0 = w0 >> 4;
  const uint32_t nb = ((uint32_t)o + Q + 15u) >> 4;
  float best = -INFINITY, second = -INFINITY;
  uint32_t arg = 0xffffffffu;
  bool nan = false;
  for (uint32_t k = lane; k < nb; k += 64u) {
    const int32_t q0 = 16 * (int32_t)k - o;
    float th[16];
    theta_chunk(k, q0, th);
    uint32_t blk[16];
    chacha_block<8>(key, b0 + k, blk);
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const int32_t q = q0 + t;
      const float v = (q >= 0 && q < (int32_t)Q) ? th[t] + gumbel_fast(blk[t]) : -INFINITY;
      nan = nan || v != v;
      const bool gt = v > best;
      second = __builtin_amdgcn_fmed3f(v, best, second);
      arg = gt ? (uint32_t)q : arg;
      best = gt ? v : best;
    }
  }
  // the sequential scan itself (NaN compares make the merges order-dependent)
  if (__builtin_amdgcn_ballot_w64(nan) != 0u) return wide_pick(Q, w0, key, theta_chunk);
#pragma unroll
  for (int m = 32; m > 0; m >>= 1)
    top2_merge(best, second, arg, __shfl_xor(best, m), __shfl_xor(second, m), __shfl_xor(arg, m));
  if (best - second > gumbel_margin(best, second)) return arg;
  best = -INFINITY;
  arg = 0xffffffffu;
  for (uint32_t k = lane; k < nb; k += 64u) {
    const int32_t q0 = 16 * (int32_t)k - o;
    float th[16];
    theta_chunk(k, q0, th);
    uint32_t blk[16];
    chacha_block<8>(key, b0 + k, blk);
#pragma unroll
    for (int t = 0; t < 16; ++t) {
      const int32_t q = q0 + t;
      if (q >= 0 && q < (int32_t)Q) {
        const float v = th[t] + gumbel_b(blk[t]);
        if (arg == 0xffffffffu || v > best) {
          best = v;
          arg = (uint32_t)q;
        }
      }
    }
  }
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) {
    const float ob = __shfl_xor(best, m);
    const uint32_t oa = __shfl_xor(arg, m);
    const bool take = ob > best || (ob == best && oa < arg);
    best = take ? ob : best;
    arg = take ? oa : arg;
  }
  return arg;
}

}  // namespace thrml
