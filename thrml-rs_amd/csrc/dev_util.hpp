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
// keys (key_expand); the three unused words are not loaded.
__device__ __forceinline__ void load_keyx(const uint32_t *__restrict__ keys, uint32_t chain,
                                          uint32_t x[KEY_WORDS]) {
  const uint4 *k4 = reinterpret_cast<const uint4 *>(keys + (size_t)chain * KEY_WORDS);
#pragma unroll
  for (int q = 0; q < 5; ++q) {
    const uint4 v = k4[q];
    x[4 * q] = v.x; x[4 * q + 1] = v.y; x[4 * q + 2] = v.z; x[4 * q + 3] = v.w;
  }
  x[20] = keys[(size_t)chain * KEY_WORDS + 20];
  x[21] = x[22] = x[23] = 0u;
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

// The spin decision `spin_uniform(w) <= sigmoid_b(x)` of the reference rule
// u <= sigmoid(2 gamma) (crates/thrml-samplers/src/spin_gibbs.rs:95-97),
// equal to it for every (x, w).  A hardware approximation
//   pa = 1 / (1 + 2^(-x log2 e))  (v_exp_f32, v_rcp_f32: 1 ulp each)
// differs from sigmoid_b(x) by less than 6e-7 on [-80, 80] (the rounding of
// x log2 e contributes at most p(1-p) |x| 2^-23 <= 2.5e-7 where p(1-p) is not
// negligible, the two hardware ops and sigmoid_b's own error the rest), so
// the decision is read off pa unless u lies within 2^-19 of it, and only
// those rare words (probability ~4e-6) take the exact sigmoid_b.
// (thrml_fast_math_check measures max |spin_pa(x) - sigmoid_b(x)| over every
// float in [-80, 80]; the tests require it below 2^-19.)  Clamping x to
// [-80, 80] changes no decision: sigmoid_b is 1 above 80 and below 2^-24
// (the smallest nonzero uniform) under -80.
__device__ __forceinline__ float spin_pa(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.44269504f));
}

__device__ __forceinline__ bool spin_decision(float x, uint32_t w) {
  x = x > 80.0f ? 80.0f : x;
  x = x < -80.0f ? -80.0f : x;
  const float u = spin_uniform(w);
  const float pa = spin_pa(x);
  if (u <= pa - 0x1p-19f) return true;
  if (u > pa + 0x1p-19f) return false;
  return u <= sigmoid_b(x);
}

// Gumbel score of a keystream word from the hardware logarithm (v_log_f32):
// -ln(-ln u) with u = gumbel_uniform(w).  u takes 2^23 values, and over all
// of them |gumbel_fast(w) - gumbel_b(w)| <= 1.91e-6 (measured exhaustively by
// thrml_fast_math_check; the tests require GUMBEL_FAST_ERR).  A categorical
// draw keeps the fast argmax when its top two scores are further apart than
// gumbel_margin, which then makes it equal to the exact argmax; otherwise
// the site is drawn again with gumbel_b.
constexpr float GUMBEL_FAST_ERR = 4e-6f;

__device__ __forceinline__ float gumbel_fast(uint32_t w) {
  const float t = __builtin_amdgcn_logf(gumbel_uniform(w)) * -0.693147182f;
  return __builtin_amdgcn_logf(t) * -0.693147182f;
}

// fl(theta + g) and fl(theta + gumbel_fast) differ by at most
// GUMBEL_FAST_ERR + ulp(v) <= GUMBEL_FAST_ERR + |v| 2^-23 for each score v,
// so a gap above twice that (with the ulp bound doubled) fixes the argmax.
__device__ __forceinline__ float gumbel_margin(float best, float second) {
  return 2.0f * GUMBEL_FAST_ERR + (fabsf(best) + fabsf(second)) * 0x1p-22f;
}

}  // namespace thrml
