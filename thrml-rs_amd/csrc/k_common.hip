// k_common.hip -- key schedule, state import/export, moment accumulation,
// hinton initialisation and the kernel-level exports.
#include <cstring>

#include "dev_util.hpp"
#include "internal.hpp"

namespace thrml {

static inline uint32_t cdiv(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

// ---------------------------------------------------------------------------
// Key schedule.  Chain c's key is RngKey::split(root, C)[c]; below it the
// reference's tree of splits (crates/thrml-samplers/src/sampling.rs) gives
// the key of every sweep:
//   run_blocks(key, n_iters)           sweep s: split(n_iters)[s]       (:93)
//   sample_with_observation(key, ...)  (wk, sk) = key.split_two()      (:189)
//     warm-up sweep w:                 split(wk, n_warmup)[w]
//     sample i (of n_samples-1), step t: split(split(sk, n_samples-1)[i],
//                                          steps_per_sample)[t]          (:222,:264)
// and sample_blocks splits a sweep key into one key per block (:37).  The
// stored value is the seed_from_u64 expansion of the block key: the ChaCha8
// key of the per-site uniform stream, stored expanded (key_expand).  Output
// layout keys[s - s0][b][c_pad][KEY_WORDS].
__device__ uint64_t sweep_key(const KeyPlan &kp, uint64_t chain_key, uint64_t s) {
  if (kp.mode == 0) return split_at(chain_key, kp.n_iters, s);
  if (s < kp.n_warmup) return split_at(split_at(chain_key, 2, 0), kp.n_warmup, s);
  s -= kp.n_warmup;
  const uint64_t i = s / kp.steps, t = s - i * kp.steps;
  const uint64_t ks = split_at(split_at(chain_key, 2, 1), kp.n_samples - 1, i);
  return split_at(ks, kp.steps, t);
}

__global__ void key_schedule_kernel(KeyPlan kp, uint64_t s0, uint32_t n_sweeps,
                                    uint32_t *__restrict__ keys) {
  const uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t total = (uint64_t)n_sweeps * kp.n_blocks * kp.C_pad;
  if (tid >= total) return;
  const uint32_t c = (uint32_t)(tid % kp.C_pad);
  const uint64_t rest = tid / kp.C_pad;
  const uint32_t b = (uint32_t)(rest % kp.n_blocks);
  const uint64_t s = s0 + rest / kp.n_blocks;
  uint4 *o = reinterpret_cast<uint4 *>(keys + tid * KEY_WORDS);
  uint32_t x[KEY_WORDS];
#pragma unroll
  for (int i = 0; i < KEY_WORDS; ++i) x[i] = 0u;
  if (c < kp.C) {
    const uint64_t k = split_at(sweep_key(kp, split_at(kp.root, kp.C, c), s), kp.n_blocks, b);
    key_expand(seed_from_u64(k).k, x);
  }
#pragma unroll
  for (int q = 0; q < KEY_WORDS / 4; ++q) o[q] = make_uint4(x[4 * q], x[4 * q + 1], x[4 * q + 2], x[4 * q + 3]);
}

int launch_key_schedule(thrml_ctx *ctx, const KeyPlan &kp, uint64_t s0, uint32_t n_sweeps,
                        uint32_t *d_keys) {
  if (n_sweeps == 0) return THRML_OK;
  const uint64_t total = (uint64_t)n_sweeps * kp.n_blocks * kp.C_pad;
  hipLaunchKernelGGL(key_schedule_kernel, dim3(cdiv(total, 256)), dim3(256), 0, ctx->stream, kp,
                     s0, n_sweeps, d_keys);
  THRML_HIP(hipGetLastError());
  return THRML_OK;
}

// ---------------------------------------------------------------------------
// State import: src[c][i] (u8 or f32) of block b -> bit planes.  One wave per
// (group, 64-site chunk); lane = chain.  A spin must be 0 or 1 (u8), or 0.0 or
// 1.0 (f32); any other value is stored as 0 and raises *bad.
__global__ void pack_kernel(const void *__restrict__ src, int dtype, uint32_t C, uint32_t n_b,
                            uint32_t planes, uint64_t *__restrict__ words, uint64_t plane_stride,
                            uint64_t blk_off, uint32_t n_chunks, uint32_t G,
                            uint32_t *__restrict__ bad) {
  const uint32_t wave = blockIdx.x * 4u + (threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t g = wave / n_chunks, chunk = wave % n_chunks;
  if (g >= G || (uint64_t)chunk * 64u >= n_b) return;
  const uint32_t c = g * 64u + lane;
  const uint32_t i_end = min(n_b, (chunk + 1u) * 64u);
  for (uint32_t i = chunk * 64u; i < i_end; ++i) {
    uint32_t v = 0;
    if (c < C) {
      const size_t off = (size_t)c * n_b + i;
      bool ok;
      if (dtype == THRML_DTYPE_U8) {
        v = reinterpret_cast<const uint8_t *>(src)[off];
        ok = v <= 1u;
      } else {
        const float x = reinterpret_cast<const float *>(src)[off];
        ok = x == 0.0f || x == 1.0f;
        v = x == 1.0f ? 1u : 0u;
      }
      if (!ok) {
        v = 0u;
        *bad = 1u;
      }
    }
    for (uint32_t pl = 0; pl < planes; ++pl) {
      const uint64_t m = __builtin_amdgcn_ballot_w64((v >> pl) & 1u);
      if (lane == 0) words[(size_t)(g * planes + pl) * plane_stride + blk_off + i] = m;
    }
  }
}

__global__ void unpack_kernel(void *__restrict__ dst, int dtype, uint32_t C, uint32_t n_b,
                              uint32_t planes, const uint64_t *__restrict__ words,
                              uint64_t plane_stride, uint64_t blk_off, uint32_t n_chunks,
                              uint32_t G) {
  const uint32_t wave = blockIdx.x * 4u + (threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t g = wave / n_chunks, chunk = wave % n_chunks;
  if (g >= G || (uint64_t)chunk * 64u >= n_b) return;
  const uint32_t c = g * 64u + lane;
  const uint32_t i_end = min(n_b, (chunk + 1u) * 64u);
  for (uint32_t i = chunk * 64u; i < i_end; ++i) {
    uint32_t v = 0;
    for (uint32_t pl = 0; pl < planes; ++pl) {
      const uint64_t w = words[(size_t)(g * planes + pl) * plane_stride + blk_off + i];
      v |= (uint32_t)((w >> lane) & 1u) << pl;
    }
    if (c < C) {
      const size_t off = (size_t)c * n_b + i;
      if (dtype == THRML_DTYPE_U8)
        reinterpret_cast<uint8_t *>(dst)[off] = (uint8_t)v;
      else
        reinterpret_cast<float *>(dst)[off] = (float)v;
    }
  }
}

// Import check before any write: raises *bad if some value of the caller's
// block is not a state value (0..q-1 as u8, or the floats 0.0..q-1.0).
__global__ void import_check_kernel(const void *__restrict__ src, int dtype, uint64_t n,
                                    uint32_t q, uint32_t *__restrict__ bad) {
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n) return;
  bool ok;
  if (dtype == THRML_DTYPE_U8) {
    ok = reinterpret_cast<const uint8_t *>(src)[t] < q;
  } else {
    const float x = reinterpret_cast<const float *>(src)[t];
    ok = x >= 0.0f && x < (float)q && x == __builtin_floorf(x);
  }
  if (!ok) *bad = 1u;
}

int launch_import_check(thrml_ctx *ctx, const void *d_src, int dtype, uint64_t n, uint32_t q,
                        uint32_t *d_bad) {
  if (n == 0) return THRML_OK;
  const uint64_t nb = (n + 255) / 256;
  if (nb > 0x7fffffffull) return fail(THRML_EUNSUPPORTED, "block too large to import");
  hipLaunchKernelGGL(import_check_kernel, dim3((uint32_t)nb), dim3(256), 0, ctx->stream, d_src,
                     dtype, n, q, d_bad);
  THRML_HIP(hipGetLastError());
  return THRML_OK;
}

int launch_pack(thrml_state *st, uint32_t b, const void *d_src, int dtype, uint32_t *d_bad) {
  thrml_prog *p = st->prog;
  const uint32_t n_b = (uint32_t)(p->blk_off[b + 1] - p->blk_off[b]);
  const uint32_t n_chunks = cdiv(n_b, 64);
  const uint32_t waves = n_chunks * st->G;
  hipLaunchKernelGGL(pack_kernel, dim3(cdiv(waves, 4)), dim3(256), 0, p->ctx->stream, d_src, dtype,
                     st->C, n_b, p->planes, st->words.as<uint64_t>(), (uint64_t)p->n_total,
                     (uint64_t)p->blk_off[b], n_chunks, st->G, d_bad);
  THRML_HIP(hipGetLastError());
  return THRML_OK;
}

int launch_unpack(thrml_state *st, uint32_t b, void *d_dst, int dtype) {
  thrml_prog *p = st->prog;
  const uint32_t n_b = (uint32_t)(p->blk_off[b + 1] - p->blk_off[b]);
  const uint32_t n_chunks = cdiv(n_b, 64);
  const uint32_t waves = n_chunks * st->G;
  hipLaunchKernelGGL(unpack_kernel, dim3(cdiv(waves, 4)), dim3(256), 0, p->ctx->stream, d_dst,
                     dtype, st->C, n_b, p->planes, st->words.as<uint64_t>(), (uint64_t)p->n_total,
                     (uint64_t)p->blk_off[b], n_chunks, st->G);
  THRML_HIP(hipGetLastError());
  return THRML_OK;
}

// ---------------------------------------------------------------------------
// Moment accumulation (MomentAccumulatorObserver::observe,
// crates/thrml-observers/src/moment.rs:157-237): per observation,
//   ones[k] += #chains with s = 1 at node k,
//   diff[k] += #chains with s_a != s_b for pair k,
// so that sum_c t = 2*ones - C*n_obs and sum_c t_a t_b = C*n_obs - 2*diff.
__global__ void moments_kernel(const uint64_t *__restrict__ words, uint64_t plane_stride,
                               uint32_t G, uint32_t C, const uint32_t *__restrict__ npos,
                               uint64_t n1, const uint32_t *__restrict__ ppos, uint64_t n2,
                               uint32_t *__restrict__ ones, uint32_t *__restrict__ diff) {
  const uint64_t tid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (tid < n1) {
    const uint32_t pos = npos[tid];
    uint32_t s = 0;
    for (uint32_t g = 0; g < G; ++g) {
      uint64_t w = words[(size_t)g * plane_stride + pos];
      const uint32_t rem = C - g * 64u;
      if (rem < 64u) w &= (1ull << rem) - 1ull;
      s += (uint32_t)__builtin_popcountll(w);
    }
    ones[tid] += s;
  } else if (tid < n1 + n2) {
    const uint64_t k = tid - n1;
    const uint32_t pa = ppos[2 * k], pb = ppos[2 * k + 1];
    uint32_t s = 0;
    for (uint32_t g = 0; g < G; ++g) {
      uint64_t w = words[(size_t)g * plane_stride + pa] ^ words[(size_t)g * plane_stride + pb];
      const uint32_t rem = C - g * 64u;
      if (rem < 64u) w &= (1ull << rem) - 1ull;
      s += (uint32_t)__builtin_popcountll(w);
    }
    diff[k] += s;
  }
}

int launch_moments(thrml_state *st, const uint32_t *d_npos, uint64_t n1, const uint32_t *d_ppos,
                   uint64_t n2, uint32_t *d_ones, uint32_t *d_diff) {
  thrml_prog *p = st->prog;
  const uint64_t total = n1 + n2;
  if (total == 0) return THRML_OK;
  hipEvent_t t0 = nullptr;
  if (p->ctx->time_begin(1, &t0)) return THRML_EHIP;
  hipLaunchKernelGGL(moments_kernel, dim3(cdiv(total, 256)), dim3(256), 0, p->ctx->stream,
                     st->words.as<uint64_t>(), (uint64_t)p->n_total, st->G, st->C, d_npos, n1,
                     d_ppos, n2, d_ones, d_diff);
  THRML_HIP(hipGetLastError());
  return p->ctx->time_end(1, t0);
}

// One observation of a general moment observer (moment.rs:153-231): thread
// r adds sum over chains of prod f(x) over row r's positions.  Spin words
// (64 chains per word): with f = 2s - 1 the product is -1 where an odd
// number of the row's spins are down, so the row's sum over a word is
// (chains) - 2 popcount(xor of the inverted words); with f = s it is the
// popcount of the words' AND.  Byte states: the product per chain in int64.
// One wave per moment row: lanes over the chain groups (bit-packed spin
// states) or over the chains (byte states, so a wave reads 64 consecutive
// bytes of a position), then a wave sum that lane 0 adds to the row's total.
__global__ __launch_bounds__(256) void observe_kernel(
    const uint64_t *__restrict__ words, const uint8_t *__restrict__ cat,
    const uint16_t *__restrict__ cat16, uint64_t plane_stride,
    uint32_t G, uint32_t C, uint32_t Cp, const uint64_t *__restrict__ row_off,
    const uint32_t *__restrict__ pos, uint64_t n_rows, int transform, int64_t *__restrict__ acc) {
  const uint64_t r = (uint64_t)blockIdx.x * 4u + (threadIdx.x >> 6);  // wave-uniform
  const uint32_t lane = threadIdx.x & 63u;
  if (r >= n_rows) return;
  const uint64_t a = row_off[r], b = row_off[r + 1];
  int64_t sum = 0;
  if (words) {
    for (uint32_t g = lane; g < G; g += 64u) {
      const uint32_t rem = C - g * 64u;
      const uint64_t valid = rem < 64u ? (1ull << rem) - 1ull : ~0ull;
      uint64_t m = transform ? 0ull : ~0ull;
      for (uint64_t k = a; k < b; ++k) {
        const uint64_t w = words[(size_t)g * plane_stride + pos[k]];
        m = transform ? (m ^ ~w) : (m & w);
      }
      const int64_t n = __builtin_popcountll(valid);
      sum += transform ? n - 2 * (int64_t)__builtin_popcountll(m & valid)
                       : (int64_t)__builtin_popcountll(m & valid);
    }
  } else {
    // the observer's creation bounds every row's product (and the run its
    // sum over chains and observations) below 2^63
    for (uint32_t c = lane; c < C; c += 64u) {
      int64_t prod = 1;
      for (uint64_t k = a; k < b; ++k) {
        const size_t at = (size_t)pos[k] * Cp + c;
        const int64_t x = cat16 ? (int64_t)cat16[at] : (int64_t)cat[at];
        prod *= transform ? 2 * x - 1 : x;
      }
      sum += prod;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  if (lane == 0u) acc[r] += sum;
}

int launch_observe(thrml_state *st, thrml_observer *obs) {
  thrml_prog *p = st->prog;
  if (obs->n_rows == 0) return THRML_OK;
  const bool bytes = byte_layout(p);
  hipLaunchKernelGGL(observe_kernel, dim3(cdiv(obs->n_rows, 4)), dim3(256), 0, p->ctx->stream,
                     bytes ? nullptr : st->words.as<uint64_t>(),
                     bytes && p->cat_bytes == 1 ? st->cat.as<uint8_t>() : nullptr,
                     bytes && p->cat_bytes == 2 ? st->cat.as<uint16_t>() : nullptr,
                     (uint64_t)p->n_total, st->G, st->C,
                     st->Cp, obs->row_off.as<uint64_t>(), obs->pos.as<uint32_t>(), obs->n_rows,
                     obs->transform ? 1 : 0, obs->acc.as<int64_t>());
  THRML_HIP(hipGetLastError());
  return THRML_OK;
}

// Folds u32 observation counters into u64 totals and clears them.
__global__ void fold_counts_kernel(uint32_t *__restrict__ cnt, uint64_t *__restrict__ acc,
                                   uint64_t n) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  acc[i] += cnt[i];
  cnt[i] = 0u;
}

// Final sums in the caller's order: sum over chains and observations of t_i
// (2*ones - C*n_obs) and of t_a*t_b (C*n_obs - 2*diff), t = 2s - 1.
__global__ void finalize_moments_kernel(const uint32_t *__restrict__ cnt1,
                                        const uint64_t *__restrict__ acc1,
                                        const uint32_t *__restrict__ slot1, uint64_t n1,
                                        const uint32_t *__restrict__ cnt2,
                                        const uint64_t *__restrict__ acc2,
                                        const uint32_t *__restrict__ slot2, uint64_t n2,
                                        int64_t cn, int64_t *__restrict__ out1,
                                        int64_t *__restrict__ out2) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n1) {
    const uint32_t s = slot1 ? slot1[i] : (uint32_t)i;
    out1[i] = 2 * (int64_t)(acc1[s] + cnt1[s]) - cn;
  } else if (i < n1 + n2) {
    const uint64_t k = i - n1;
    const uint32_t s = slot2 ? slot2[k] : (uint32_t)k;
    out2[k] = cn - 2 * (int64_t)(acc2[s] + cnt2[s]);
  }
}

int launch_fold_counts(thrml_ctx *ctx, uint32_t *cnt, uint64_t *acc, uint64_t n) {
  if (n == 0) return THRML_OK;
  hipLaunchKernelGGL(fold_counts_kernel, dim3(cdiv(n, 256)), dim3(256), 0, ctx->stream, cnt, acc, n);
  THRML_HIP(hipGetLastError());
  return THRML_OK;
}

int launch_finalize_moments(thrml_ctx *ctx, const uint32_t *cnt1, const uint64_t *acc1,
                            const uint32_t *slot1, uint64_t n1, const uint32_t *cnt2,
                            const uint64_t *acc2, const uint32_t *slot2, uint64_t n2, int64_t cn,
                            int64_t *out1, int64_t *out2) {
  if (n1 + n2 == 0) return THRML_OK;
  hipLaunchKernelGGL(finalize_moments_kernel, dim3(cdiv(n1 + n2, 256)), dim3(256), 0, ctx->stream,
                     cnt1, acc1, slot1, n1, cnt2, acc2, slot2, n2, cn, out1, out2);
  THRML_HIP(hipGetLastError());
  return THRML_OK;
}

// ---------------------------------------------------------------------------
// hinton_init (crates/thrml-models/src/ising.rs:602-673) of free block b:
// entry (c, i) of the [C, n_b] uniform tensor is keystream word c*n_b + i of
// the block key; s = (word <= threshold(sigmoid(b_i * beta))).
__global__ void hinton_kernel(const uint32_t *__restrict__ key8, const float *__restrict__ prob,
                              uint32_t C, uint32_t n_b, uint64_t *__restrict__ words,
                              uint64_t group_stride, uint64_t blk_off, uint32_t n_seg,
                              uint32_t n_tasks) {
  const uint32_t task = blockIdx.x * 4u + (threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  if (task >= n_tasks) return;
  const uint32_t g = task / n_seg, seg = task % n_seg;
  const uint32_t c = g * 64u + lane;
  uint64_t *__restrict__ out = words + (size_t)g * group_stride + blk_off;
  Key8 key;
#pragma unroll
  for (int i = 0; i < 8; ++i) key.k[i] = key8[i];
  const uint32_t i0 = seg * 16u;
  const uint64_t w0 = (uint64_t)c * n_b + i0;
  uint32_t a[16], bb[16];
  chacha_block<8>(key.k, w0 >> 4, a);
  chacha_block<8>(key.k, (w0 >> 4) + 1, bb);
  const uint32_t sh = (uint32_t)(w0 & 15u);
#pragma unroll 1
  for (uint32_t k = 0; k < 16u; ++k) {
    const uint32_t i = i0 + k;
    if (i >= n_b) break;
    const uint32_t pos = sh + k;  // 0..30
    uint32_t wd = 0;
#pragma unroll
    for (uint32_t t = 0; t < 16u; ++t) {
      wd = (pos == t) ? a[t] : wd;
      wd = (pos == t + 16u) ? bb[t] : wd;
    }
    const bool up = (c < C) && (wd <= word_threshold(prob[i]));
    const uint64_t m = __builtin_amdgcn_ballot_w64(up);
    if (lane == 0) out[i] = m;
  }
}

int launch_hinton(thrml_prog *p, thrml_state *st, uint32_t b, const uint32_t *d_key8,
                  const float *d_prob) {
  const uint32_t n_b = (uint32_t)(p->blk_off[b + 1] - p->blk_off[b]);
  const uint32_t n_seg = cdiv(n_b, 16);
  const uint32_t n_tasks = n_seg * st->G;
  hipLaunchKernelGGL(hinton_kernel, dim3(cdiv(n_tasks, 4)), dim3(256), 0, p->ctx->stream, d_key8,
                     d_prob, st->C, n_b, st->words.as<uint64_t>(),
                     (uint64_t)p->planes * p->n_total, (uint64_t)p->blk_off[b], n_seg, n_tasks);
  THRML_HIP(hipGetLastError());
  return THRML_OK;
}

// ---------------------------------------------------------------------------
// FusedKernelBackend counterparts (crates/thrml-kernels/src/lib.rs:55-106).
__global__ void sigmoid_bernoulli_kernel(const float *__restrict__ g, const float *__restrict__ u,
                                         float *__restrict__ o, uint64_t n) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  // the inputs are arbitrary floats: the full-range sigmoid, so that a
  // pre-activation below -40 gives probability 0 (u = 0 then samples 0)
  const float prob = sigmoid_full(2.0f * g[i]);
  o[i] = (u[i] < prob) ? 1.0f : 0.0f;  // strict, as sigmoid_bernoulli/kernel.rs:53
}

// gumbel = 0 - log(0 - log(u)) and perturbed = logit + gumbel, as written in
// gumbel_argmax/kernel.rs:61-75, with the full-range log: u = 0 scores -inf
// (never taken after index 0), u = 1 scores +inf, a NaN score never wins.
__device__ __forceinline__ float gumbel_score(float logit, float u) {
  return logit + (0.0f - log_full(0.0f - log_full(u)));
}

__global__ void gumbel_argmax_kernel(const float *__restrict__ l, const float *__restrict__ u,
                                     int32_t *__restrict__ o, uint64_t n, uint32_t q) {
  const uint64_t r = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= n) return;
  const float *lr = l + r * q;
  const float *ur = u + r * q;
  float best = gumbel_score(lr[0], ur[0]);
  int32_t arg = 0;
  for (uint32_t k = 1; k < q; ++k) {
    const float v = gumbel_score(lr[k], ur[k]);
    if (v > best) {  // first maximum, gumbel_argmax/kernel.rs:81-83
      best = v;
      arg = (int32_t)k;
    }
  }
  o[r] = arg;
}

int launch_sigmoid_bernoulli(thrml_ctx *ctx, const float *g, const float *u, float *o, uint64_t n) {
  if (n == 0) return THRML_OK;
  hipLaunchKernelGGL(sigmoid_bernoulli_kernel, dim3(cdiv(n, 256)), dim3(256), 0, ctx->stream, g, u,
                     o, n);
  THRML_HIP(hipGetLastError());
  return THRML_OK;
}

int launch_gumbel_argmax(thrml_ctx *ctx, const float *l, const float *u, int32_t *o, uint64_t n,
                         uint32_t q) {
  if (n == 0) return THRML_OK;
  hipLaunchKernelGGL(gumbel_argmax_kernel, dim3(cdiv(n, 256)), dim3(256), 0, ctx->stream, l, u, o,
                     n, q);
  THRML_HIP(hipGetLastError());
  return THRML_OK;
}

// batch_gather_fused (batch_gather/kernel.rs, launched by batch_gather/forward.rs):
// out[b] = weights[b * batch_stride + sum_i u32(indices[b][i]) * strides[i]],
// the index arithmetic in u32 as the reference's (wrapping).  A linear index
// at or past n_weights reads 0.0 (one of the values a bounds-checked read of
// the reference's buffer may give) instead of leaving the array.
__global__ void batch_gather_kernel(const float *__restrict__ w, uint64_t n_w,
                                    const int32_t *__restrict__ idx, uint64_t batch, uint32_t n_idx,
                                    BatchGatherStrides st, float *__restrict__ out) {
  const uint64_t b = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  uint32_t lin = (uint32_t)b * st.batch_stride;
  const int32_t *ib = idx + b * n_idx;
  for (uint32_t i = 0; i < n_idx; ++i) lin += (uint32_t)ib[i] * st.s[i];
  out[b] = lin < n_w ? w[lin] : 0.0f;
}

int launch_batch_gather(thrml_ctx *ctx, const float *w, uint64_t n_w, const int32_t *idx,
                        uint64_t batch, uint32_t n_idx, const BatchGatherStrides &st, float *out) {
  if (batch == 0) return THRML_OK;
  hipLaunchKernelGGL(batch_gather_kernel, dim3(cdiv(batch, 256)), dim3(256), 0, ctx->stream, w,
                     n_w, idx, batch, n_idx, st, out);
  THRML_HIP(hipGetLastError());
  return THRML_OK;
}

// ---------------------------------------------------------------------------
// Self-check of the hardware-math fast paths (no counterpart in the
// reference): thread i takes uniform numerator 2i+1 for the Gumbel bound and
// every 2^23-th float of [0, 40] (both signs) for the spin decision's two
// relative errors, against double-precision references.
// bits of the smallest float >= v (v >= 0), so that no bound is understated
__device__ __forceinline__ uint32_t f32_bits_up(double v) {
  const float f = (float)v;
  return __builtin_bit_cast(uint32_t, f) + ((double)f < v ? 1u : 0u);
}

__global__ void fast_math_check_kernel(uint32_t *__restrict__ out) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (1u << 23)) return;
  const uint32_t w = (2u * i + 1u) << 8;
  const float eg = fabsf(gumbel_fast(w) - gumbel_b(w));
  double ee = 0.0, es = 0.0;
  for (uint32_t b = i; b <= 0x42200000u; b += (1u << 23)) {  // bits of 40.0f
    const float gp = __builtin_bit_cast(float, b);
#pragma unroll
    for (int sgn = 0; sgn < 2; ++sgn) {
      const float g = sgn ? -gp : gp;
      const double en = exp(-2.0 * (double)g);
      ee = fmax(ee, fabs((double)spin_exp_neg(g) - en) / en);
      const double sig = 1.0 / (1.0 + en);
      es = fmax(es, fabs((double)sigmoid_b(2.0f * g) - sig) / sig);
    }
  }
  // non-negative floats order as their bits
  atomicMax(out + 0, __builtin_bit_cast(uint32_t, eg));
  atomicMax(out + 1, f32_bits_up(ee));
  atomicMax(out + 2, f32_bits_up(es));
}

int launch_fast_math_check(thrml_ctx *ctx, float out[3]) {
  uint32_t *d = nullptr;
  THRML_HIP(hipMalloc(&d, 12));
  uint32_t h[3] = {0u, 0u, 0u};
  hipError_t e = hipMemcpyAsync(d, h, 12, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) {
    hipLaunchKernelGGL(fast_math_check_kernel, dim3((1u << 23) / 256), dim3(256), 0, ctx->stream, d);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipMemcpyAsync(h, d, 12, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  (void)hipFree(d);
  if (e != hipSuccess) return hip_fail(e, "fast math check");
  std::memcpy(out, h, 12);
  return THRML_OK;
}

}  // namespace thrml
