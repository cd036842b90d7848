/*
 * orc_rng.c -- oracle restatement of RngKey (crates/thrml-samplers/src/rng.rs).
 *
 * TEST INFRASTRUCTURE ONLY (see thrml_oracle.h).
 *
 * RngKey::split (rng.rs:20-38) calls ChaCha8Rng::seed_from_u64 (rand_chacha
 * 0.3.1 / rand_core 0.6.4, pinned at Cargo.lock:3353-3381, not vendored in the
 * reference) and then next_u64 n times.  Restated from the crates' published
 * algorithm:
 *   - seed_from_u64: a PCG32 generator (multiplier 6364136223846793005,
 *     increment 11634580027462260723, XSH-RR output) advanced once per 4-byte
 *     chunk; the 32-byte seed is the 8 little-endian outputs;
 *   - ChaCha8Rng::from_seed: key = seed, 64-bit block counter (words 12,13)
 *     starting at 0, 64-bit stream id (words 14,15) = 0;
 *   - the block RNG buffers consecutive blocks; next_u64 returns
 *     word[2j] | word[2j+1] << 32 (the index is always even when only
 *     next_u64 is called).
 * The ChaCha block function is pinned by RFC 8439 vectors (rounds = 20) in
 * tests/test_oracle_rng.py; the round count is the only change for ChaCha8.
 */
#include "thrml_oracle.h"

#define ROTL32(x, n) (((x) << (n)) | ((x) >> (32 - (n))))

static void quarter(uint32_t *s, int a, int b, int c, int d) {
  s[a] += s[b]; s[d] ^= s[a]; s[d] = ROTL32(s[d], 16);
  s[c] += s[d]; s[b] ^= s[c]; s[b] = ROTL32(s[b], 12);
  s[a] += s[b]; s[d] ^= s[a]; s[d] = ROTL32(s[d], 8);
  s[c] += s[d]; s[b] ^= s[c]; s[b] = ROTL32(s[b], 7);
}

void orc_chacha_block(const uint32_t key[8], uint64_t counter, uint64_t stream,
                      int rounds, uint32_t out[16]) {
  uint32_t in[16], x[16];
  in[0] = 0x61707865u; /* "expa" */
  in[1] = 0x3320646eu; /* "nd 3" */
  in[2] = 0x79622d32u; /* "2-by" */
  in[3] = 0x6b206574u; /* "te k" */
  for (int i = 0; i < 8; i++) in[4 + i] = key[i];
  in[12] = (uint32_t)counter;
  in[13] = (uint32_t)(counter >> 32);
  in[14] = (uint32_t)stream;
  in[15] = (uint32_t)(stream >> 32);
  for (int i = 0; i < 16; i++) x[i] = in[i];
  for (int r = 0; r < rounds; r += 2) {
    quarter(x, 0, 4, 8, 12);
    quarter(x, 1, 5, 9, 13);
    quarter(x, 2, 6, 10, 14);
    quarter(x, 3, 7, 11, 15);
    quarter(x, 0, 5, 10, 15);
    quarter(x, 1, 6, 11, 12);
    quarter(x, 2, 7, 8, 13);
    quarter(x, 3, 4, 9, 14);
  }
  for (int i = 0; i < 16; i++) out[i] = x[i] + in[i];
}

void orc_seed_from_u64(uint64_t state, uint32_t key_out[8]) {
  const uint64_t mul = 6364136223846793005ull;
  const uint64_t inc = 11634580027462260723ull;
  for (int i = 0; i < 8; i++) {
    state = state * mul + inc;
    uint32_t xorshifted = (uint32_t)(((state >> 18) ^ state) >> 27);
    uint32_t rot = (uint32_t)(state >> 59);
    key_out[i] = (xorshifted >> rot) | (xorshifted << ((32u - rot) & 31u));
  }
}

uint32_t orc_stream_word(const uint32_t key8[8], uint64_t w) {
  uint32_t blk[16];
  orc_chacha_block(key8, w >> 4, 0, 8, blk);
  return blk[w & 15];
}

void orc_rng_split(uint64_t key, size_t n, uint64_t *out) {
  if (n == 0) return;
  if (n == 1) {
    out[0] = key;
    return;
  }
  uint32_t k8[8], blk[16];
  orc_seed_from_u64(key, k8);
  uint64_t cur_block = (uint64_t)-1;
  for (size_t i = 0; i < n; i++) {
    uint64_t w = 2 * (uint64_t)i;
    if ((w >> 4) != cur_block) {
      cur_block = w >> 4;
      orc_chacha_block(k8, cur_block, 0, 8, blk);
    }
    out[i] = (uint64_t)blk[w & 15] | ((uint64_t)blk[(w & 15) + 1] << 32);
  }
}
