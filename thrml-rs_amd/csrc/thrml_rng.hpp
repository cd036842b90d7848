// thrml_rng.hpp -- RngKey splitting and the per-site ChaCha8 stream, for host
// and device.
//
// RngKey::split (crates/thrml-samplers/src/rng.rs:20-38) is
//   n == 0 -> [], n == 1 -> [key],
//   else ChaCha8Rng::seed_from_u64(key) followed by n calls of next_u64.
// rand_core 0.6's seed_from_u64 expands a u64 into the 32-byte ChaCha key with
// a PCG32 generator (LCG multiplier 6364136223846793005, increment
// 11634580027462260723, XSH-RR output), one output per 4-byte key word.
// rand_chacha 0.3's ChaCha8Rng keystream is the ChaCha block function with 8
// rounds, 64-bit block counter in state words 12-13 starting at 0 and a zero
// stream id in words 14-15; next_u64 = w[2j] | w[2j+1] << 32.  Because the
// keystream is counter based, element i of split(key, n) is computed here
// directly from block i/8 (`split_at`) without materialising the others.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define THRML_HD __host__ __device__ __forceinline__
#else
#define THRML_HD inline
#endif

namespace thrml {

THRML_HD uint32_t rotl32(uint32_t x, int n) { return (x << n) | (x >> (32 - n)); }

// Expanded ChaCha8 key: the 8 key words after seed_from_u64.
struct Key8 {
  uint32_t k[8];
};

THRML_HD Key8 seed_from_u64(uint64_t s) {
  Key8 out;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    s = s * 6364136223846793005ull + 11634580027462260723ull;
    uint32_t xs = (uint32_t)(((s >> 18) ^ s) >> 27);
    uint32_t rot = (uint32_t)(s >> 59);
    out.k[i] = (xs >> rot) | (xs << ((32u - rot) & 31u));
  }
  return out;
}

// ChaCha quarter round on four words held in registers.
#define THRML_QR(a, b, c, d)                 \
  do {                                       \
    a += b; d ^= a; d = thrml::rotl32(d, 16); \
    c += d; b ^= c; b = thrml::rotl32(b, 12); \
    a += b; d ^= a; d = thrml::rotl32(d, 8);  \
    c += d; b ^= c; b = thrml::rotl32(b, 7);  \
  } while (0)

// One 16-word ChaCha block with `ROUNDS` rounds (8 for ChaCha8) for block
// counter `ctr` and stream id 0.  Fully unrolled: every word stays in a
// register.
template <int ROUNDS = 8>
THRML_HD void chacha_block(const uint32_t k[8], uint64_t ctr, uint32_t out[16]) {
  const uint32_t c0 = 0x61707865u, c1 = 0x3320646eu, c2 = 0x79622d32u, c3 = 0x6b206574u;
  uint32_t x0 = c0, x1 = c1, x2 = c2, x3 = c3;
  uint32_t x4 = k[0], x5 = k[1], x6 = k[2], x7 = k[3];
  uint32_t x8 = k[4], x9 = k[5], x10 = k[6], x11 = k[7];
  uint32_t x12 = (uint32_t)ctr, x13 = (uint32_t)(ctr >> 32), x14 = 0u, x15 = 0u;
#pragma unroll
  for (int r = 0; r < ROUNDS; r += 2) {
    THRML_QR(x0, x4, x8, x12);
    THRML_QR(x1, x5, x9, x13);
    THRML_QR(x2, x6, x10, x14);
    THRML_QR(x3, x7, x11, x15);
    THRML_QR(x0, x5, x10, x15);
    THRML_QR(x1, x6, x11, x12);
    THRML_QR(x2, x7, x8, x13);
    THRML_QR(x3, x4, x9, x14);
  }
  out[0] = x0 + c0;
  out[1] = x1 + c1;
  out[2] = x2 + c2;
  out[3] = x3 + c3;
  out[4] = x4 + k[0];
  out[5] = x5 + k[1];
  out[6] = x6 + k[2];
  out[7] = x7 + k[3];
  out[8] = x8 + k[4];
  out[9] = x9 + k[5];
  out[10] = x10 + k[6];
  out[11] = x11 + k[7];
  out[12] = x12 + (uint32_t)ctr;
  out[13] = x13 + (uint32_t)(ctr >> 32);
  out[14] = x14;
  out[15] = x15;
}

// Stream keys as stored for the sweep kernels: KEY_WORDS words per key.
// With stream id 0 and a block counter below 2^32 (word 13 = 0), three of
// the first round's four column quarter rounds, QR(1,5,9,13), QR(2,6,10,14)
// and QR(3,7,11,15), and the first addition of QR(0,4,8,12), depend on the
// key alone; so do the first addition of the diagonal QR(1,6,11,12) and the
// first three steps of QR(2,7,8,13) (a += b; d ^= a; d <<<= 16), whose
// inputs all come from those three column rounds.  They are computed once
// per key:
//   x[0..7]   the key words (the final addition needs them),
//   x[8..19]  words 1,5,9,13, 2,6,10,14, 3,7,11,15 after their first quarter round,
//   x[20]     constant 0 + key word 0,
//   x[21]     word 1 + word 6 (the diagonal round's new word 1),
//   x[22]     word 2 + word 7 (its new word 2),
//   x[23]     (word 13 ^ x[22]) <<< 16 (its new word 13).
constexpr int KEY_WORDS = 24;

THRML_HD void key_expand(const uint32_t k[8], uint32_t x[KEY_WORDS]) {
  uint32_t a1 = 0x3320646eu, b1 = k[1], c1 = k[5], d1 = 0u;
  uint32_t a2 = 0x79622d32u, b2 = k[2], c2 = k[6], d2 = 0u;
  uint32_t a3 = 0x6b206574u, b3 = k[3], c3 = k[7], d3 = 0u;
  THRML_QR(a1, b1, c1, d1);
  THRML_QR(a2, b2, c2, d2);
  THRML_QR(a3, b3, c3, d3);
  for (int i = 0; i < 8; ++i) x[i] = k[i];
  x[8] = a1; x[9] = b1; x[10] = c1; x[11] = d1;
  x[12] = a2; x[13] = b2; x[14] = c2; x[15] = d2;
  x[16] = a3; x[17] = b3; x[18] = c3; x[19] = d3;
  x[20] = 0x61707865u + k[0];
  x[21] = a1 + b2;
  x[22] = a2 + b3;
  x[23] = rotl32(d1 ^ x[22], 16);
}

// chacha_block<ROUNDS>(k, ctr) from an expanded key x (key_expand(k)), for
// ctr < 2^32: the same 16 words, 41 fewer operations.
template <int ROUNDS = 8>
THRML_HD void chacha_block_pre(const uint32_t x[KEY_WORDS], uint32_t ctr, uint32_t out[16]) {
  uint32_t x0 = x[20], x4 = x[0], x8 = x[4], x12 = ctr;
  // the rest of QR(0, 4, 8, 12) after its first addition
  x12 ^= x0; x12 = rotl32(x12, 16);
  x8 += x12; x4 ^= x8; x4 = rotl32(x4, 12);
  x0 += x4; x12 ^= x0; x12 = rotl32(x12, 8);
  x8 += x12; x4 ^= x8; x4 = rotl32(x4, 7);
  uint32_t x5 = x[9], x9 = x[10];
  uint32_t x6 = x[13], x10 = x[14], x14 = x[15];
  uint32_t x3 = x[16], x7 = x[17], x11 = x[18], x15 = x[19];
  THRML_QR(x0, x5, x10, x15);
  // QR(1, 6, 11, 12) after its first addition (x1 = x[21])
  uint32_t x1 = x[21];
  x12 ^= x1; x12 = rotl32(x12, 16);
  x11 += x12; x6 ^= x11; x6 = rotl32(x6, 12);
  x1 += x6; x12 ^= x1; x12 = rotl32(x12, 8);
  x11 += x12; x6 ^= x11; x6 = rotl32(x6, 7);
  // QR(2, 7, 8, 13) after its first three steps (x2 = x[22], x13 = x[23])
  uint32_t x2 = x[22], x13 = x[23];
  x8 += x13; x7 ^= x8; x7 = rotl32(x7, 12);
  x2 += x7; x13 ^= x2; x13 = rotl32(x13, 8);
  x8 += x13; x7 ^= x8; x7 = rotl32(x7, 7);
  THRML_QR(x3, x4, x9, x14);
#pragma unroll
  for (int r = 2; r < ROUNDS; r += 2) {
    THRML_QR(x0, x4, x8, x12);
    THRML_QR(x1, x5, x9, x13);
    THRML_QR(x2, x6, x10, x14);
    THRML_QR(x3, x7, x11, x15);
    THRML_QR(x0, x5, x10, x15);
    THRML_QR(x1, x6, x11, x12);
    THRML_QR(x2, x7, x8, x13);
    THRML_QR(x3, x4, x9, x14);
  }
  out[0] = x0 + 0x61707865u;
  out[1] = x1 + 0x3320646eu;
  out[2] = x2 + 0x79622d32u;
  out[3] = x3 + 0x6b206574u;
  out[4] = x4 + x[0];
  out[5] = x5 + x[1];
  out[6] = x6 + x[2];
  out[7] = x7 + x[3];
  out[8] = x8 + x[4];
  out[9] = x9 + x[5];
  out[10] = x10 + x[6];
  out[11] = x11 + x[7];
  out[12] = x12 + ctr;
  out[13] = x13;
  out[14] = x14;
  out[15] = x15;
}

// Same block function with an explicit stream id (used only to check the
// RFC 8439 layout, whose nonce occupies words 13-15).
template <int ROUNDS>
THRML_HD void chacha_block_stream(const uint32_t k[8], uint32_t w12, uint32_t w13,
                                  uint32_t w14, uint32_t w15, uint32_t out[16]) {
  uint32_t in[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u,
                     k[0], k[1], k[2], k[3], k[4], k[5], k[6], k[7], w12, w13, w14, w15};
  uint32_t x0 = in[0], x1 = in[1], x2 = in[2], x3 = in[3], x4 = in[4], x5 = in[5],
           x6 = in[6], x7 = in[7], x8 = in[8], x9 = in[9], x10 = in[10], x11 = in[11],
           x12 = in[12], x13 = in[13], x14 = in[14], x15 = in[15];
  for (int r = 0; r < ROUNDS; r += 2) {
    THRML_QR(x0, x4, x8, x12);
    THRML_QR(x1, x5, x9, x13);
    THRML_QR(x2, x6, x10, x14);
    THRML_QR(x3, x7, x11, x15);
    THRML_QR(x0, x5, x10, x15);
    THRML_QR(x1, x6, x11, x12);
    THRML_QR(x2, x7, x8, x13);
    THRML_QR(x3, x4, x9, x14);
  }
  uint32_t x[16] = {x0, x1, x2, x3, x4, x5, x6, x7, x8, x9, x10, x11, x12, x13, x14, x15};
  for (int i = 0; i < 16; ++i) out[i] = x[i] + in[i];
}

// Word w of the ChaCha8 keystream of an expanded key.
THRML_HD uint32_t stream_word(const Key8& key, uint64_t w) {
  uint32_t blk[16];
  chacha_block<8>(key.k, w >> 4, blk);
  uint32_t r = blk[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) r = ((w & 15u) == (uint64_t)i) ? blk[i] : r;
  return r;
}

// Element i of RngKey(key).split(n) (requires i < n).
THRML_HD uint64_t split_at(uint64_t key, uint64_t n, uint64_t i) {
  if (n == 1) return key;
  Key8 k = seed_from_u64(key);
  uint32_t blk[16];
  chacha_block<8>(k.k, i >> 3, blk);
  uint32_t j = (uint32_t)(i & 7u) * 2u;
  uint32_t lo = blk[0], hi = blk[1];
#pragma unroll
  for (int t = 1; t < 8; ++t) {
    lo = (j == 2u * t) ? blk[2 * t] : lo;
    hi = (j == 2u * t) ? blk[2 * t + 1] : hi;
  }
  return (uint64_t)lo | ((uint64_t)hi << 32);
}

}  // namespace thrml
