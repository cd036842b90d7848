// Test-only shim: the product's shared host/device headers compiled for the
// CPU, so tests can compare them bit for bit with the oracle's restatement
// (the GPU tests then compare the device build with the same oracle).
#include <stdint.h>

#include "../../thrml-rs_amd/csrc/thrml_math.hpp"
#include "../../thrml-rs_amd/csrc/thrml_rng.hpp"

extern "C" {
void shim_fastdiv(uint32_t d, const uint32_t *x, uint32_t *q, uint64_t n) {
  const thrml::FastDiv f = thrml::make_fastdiv(d);
  for (uint64_t i = 0; i < n; ++i) q[i] = thrml::fdiv(x[i], f);
}
void shim_exp(const float *x, float *y, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) y[i] = thrml::exp_b(x[i]);
}
void shim_sigmoid(const float *x, float *y, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) y[i] = thrml::sigmoid_b(x[i]);
}
void shim_log(const float *x, float *y, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) y[i] = thrml::log_b(x[i]);
}
void shim_exp_full(const float *x, float *y, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) y[i] = thrml::exp_full(x[i]);
}
void shim_sigmoid_full(const float *x, float *y, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) y[i] = thrml::sigmoid_full(x[i]);
}
void shim_log_full(const float *x, float *y, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) y[i] = thrml::log_full(x[i]);
}
void shim_gumbel(const uint32_t *w, float *y, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) y[i] = thrml::gumbel_b(w[i]);
}
void shim_threshold(const float *p, uint32_t *t, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) t[i] = thrml::word_threshold(p[i]);
}
void shim_chacha8(const uint32_t *key, uint64_t ctr, uint32_t *out) {
  thrml::chacha_block<8>(key, ctr, out);
}
void shim_chacha8_pre(const uint32_t *key, uint32_t ctr, uint32_t *out) {
  uint32_t x[thrml::KEY_WORDS];
  thrml::key_expand(key, x);
  thrml::chacha_block_pre<8>(x, ctr, out);
}
void shim_chacha_rfc(const uint32_t *key, int rounds, uint32_t w12, uint32_t w13, uint32_t w14,
                     uint32_t w15, uint32_t *out) {
  if (rounds == 20)
    thrml::chacha_block_stream<20>(key, w12, w13, w14, w15, out);
  else
    thrml::chacha_block_stream<8>(key, w12, w13, w14, w15, out);
}
void shim_seed(uint64_t s, uint32_t *k) {
  thrml::Key8 e = thrml::seed_from_u64(s);
  for (int i = 0; i < 8; ++i) k[i] = e.k[i];
}
uint64_t shim_split_at(uint64_t key, uint64_t n, uint64_t i) { return thrml::split_at(key, n, i); }
uint32_t shim_stream_word(const uint32_t *k, uint64_t w) {
  thrml::Key8 e;
  for (int i = 0; i < 8; ++i) e.k[i] = k[i];
  return thrml::stream_word(e, w);
}
}
