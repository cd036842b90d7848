// k_ising.hip -- Ising half-sweep kernels for gfx950.
//
// One launch updates one free block of every chain (the body of
// sample_single_block, crates/thrml-samplers/src/program.rs:324-393, with the
// SpinGibbsConditional update of crates/thrml-samplers/src/spin_gibbs.rs:56-100
// and :512-637 fused in, for 64 chains per wave).
//
// Work decomposition: a wave takes one chain group g (64 chains, lane l =
// chain 64g + l) and a segment of 16 consecutive block-local sites i0..i0+15.
// Lane l draws its 16 uniforms from one ChaCha8 block: block-local site i of
// the block key (c, sweep, block) takes keystream word i, i.e. word i%16 of
// block i/16.  Everything that depends only on the site (neighbour
// positions, weights, bias, table row) is wave-uniform and lives in scalar
// registers; a neighbour's 64 chain bits are one 64-bit word used directly as
// a lane mask; the 64 new bits of a site are one ballot.
//
// Workgroups are remapped so that each of the 8 XCDs (which take workgroups
// round-robin) walks a contiguous range of segments: neighbouring rows then
// share an XCD's L2.
#include "internal.hpp"
#include "thrml_math.hpp"
#include "thrml_rng.hpp"

namespace thrml {

__device__ __forceinline__ uint32_t xcd_remap(uint32_t bid, uint32_t nwg) {
  const uint32_t nx = 8;
  const uint32_t xcd = bid % nx, idx = bid / nx;
  const uint32_t per = nwg / nx, rem = nwg % nx;
  return xcd * per + (xcd < rem ? xcd : rem) + idx;
}

__device__ __forceinline__ Key8 load_key(const uint32_t *__restrict__ keys, uint32_t chain) {
  const uint4 *k4 = reinterpret_cast<const uint4 *>(keys + (size_t)chain * 8);
  const uint4 a = k4[0], b = k4[1];
  Key8 k;
  k.k[0] = a.x; k.k[1] = a.y; k.k[2] = a.z; k.k[3] = a.w;
  k.k[4] = b.x; k.k[5] = b.y; k.k[6] = b.z; k.k[7] = b.w;
  return k;
}

__device__ __forceinline__ bool lane_bit(uint64_t w) {
  return __builtin_amdgcn_inverse_ballot_w64(w);
}

// ---------------------------------------------------------------------------
// Lattice half-sweep.  table[i][cfg] is the keystream-word threshold of
// block-local site i for neighbour configuration cfg = L | R<<1 | U<<2 | D<<3
// (1 = spin up); the table was built with gamma summed in the reference's
// slot order, so the comparison `word <= table` is exactly
// `u <= sigmoid(2*gamma)`.
__global__ __launch_bounds__(256) void lattice_half_kernel(
    const uint64_t *__restrict__ other, uint64_t *__restrict__ mine,
    const uint32_t *__restrict__ table, const uint32_t *__restrict__ keys, uint32_t n_b,
    uint32_t L, uint32_t half, uint32_t par, uint64_t plane_stride, uint32_t n_seg,
    uint32_t n_tasks) {
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t task = xcd_remap(blockIdx.x, gridDim.x) * 4u + wave;
  if (task >= n_tasks) return;
  const uint32_t g = task / n_seg;
  const uint32_t seg = task - g * n_seg;
  const uint64_t *__restrict__ oth = other + (size_t)g * plane_stride;
  uint64_t *__restrict__ out = mine + (size_t)g * plane_stride;

  const uint32_t i0 = seg * 16u;
  uint32_t r = i0 / half;
  uint32_t t = i0 - r * half;

  // Phase 1: neighbour words (scalar), configuration (per lane), table
  // thresholds (vector gather within one 64-byte row).
  uint32_t thr[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const uint32_t i = i0 + k;
    uint32_t th = 0u;
    if (i < n_b) {
      const uint32_t j = 2u * t + ((r + par) & 1u);
      const uint32_t jl = (j == 0u ? L : j) - 1u;
      const uint32_t jr = (j + 1u == L) ? 0u : j + 1u;
      const uint32_t ru = (r == 0u ? L : r) - 1u;
      const uint32_t rd = (r + 1u == L) ? 0u : r + 1u;
      const uint64_t wl = oth[(size_t)r * half + (jl >> 1)];
      const uint64_t wr = oth[(size_t)r * half + (jr >> 1)];
      const uint64_t wu = oth[(size_t)ru * half + t];
      const uint64_t wd = oth[(size_t)rd * half + t];
      const uint32_t cfg = (lane_bit(wl) ? 1u : 0u) | (lane_bit(wr) ? 2u : 0u) |
                           (lane_bit(wu) ? 4u : 0u) | (lane_bit(wd) ? 8u : 0u);
      th = table[(size_t)i * 16u + cfg];
    }
    thr[k] = th;
    if (++t == half) {
      t = 0;
      ++r;
    }
  }

  // Phase 2: this lane's 16 uniforms.
  const Key8 key = load_key(keys, g * 64u + lane);
  uint32_t x[16];
  chacha_block<8>(key.k, seg, x);

  // Phase 3: decisions; lane 0 writes the 64-chain word of each site.
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    const uint32_t i = i0 + k;
    if (i < n_b) {
      const uint64_t m = __builtin_amdgcn_ballot_w64(x[k] <= thr[k]);
      if (lane == 0) out[i] = m;
    }
  }
}

// Threshold table: one thread per (site, cfg).  dir[s] in 0..3 gives the
// lattice direction (L, R, U, D) of slot s; slots are in reference order.
__global__ void lattice_table_kernel(const uint32_t *__restrict__ row_off,
                                     const uint32_t *__restrict__ dir,
                                     const float *__restrict__ w,
                                     const float *__restrict__ bias_w, uint32_t n,
                                     int has_bias, int has_edges, uint32_t *__restrict__ table) {
  const uint32_t tid = blockIdx.x * blockDim.x + threadIdx.x;
  if (tid >= n * 16u) return;
  const uint32_t p = tid >> 4, cfg = tid & 15u;
  float g = 0.0f;
  if (has_bias) g = g + bias_w[p];
  if (has_edges) {
    float acc = 0.0f;
    const uint32_t a = row_off[p], b = row_off[p + 1];
    for (uint32_t s = a; s < b; ++s) {
      const float wt = w[s];
      const float tv = ((cfg >> dir[s]) & 1u) ? wt : -wt;
      acc = (s == a) ? tv : acc + tv;
    }
    g = g + acc;
  }
  table[tid] = word_threshold(sigmoid_b(g * 2.0f));
}

// ---------------------------------------------------------------------------
// CSR half-sweep for arbitrary Ising programs.  slots[s] = {global position
// of the tail node, fl(beta*J)} in the reference's slot order (u-role edges
// ascending, then v-role edges ascending); gamma is accumulated per lane in
// that order: acc = fl(acc + (+-w)), computed as fma(+-1, w, acc).
__global__ __launch_bounds__(256) void csr_half_kernel(
    const uint64_t *__restrict__ words_in, uint64_t *__restrict__ out_words,
    const uint32_t *__restrict__ row_off, const uint2 *__restrict__ slots,
    const float *__restrict__ bias_w, const uint32_t *__restrict__ keys, uint32_t n_b,
    uint32_t blk_off, uint64_t plane_stride, uint64_t out_stride, uint32_t n_seg,
    uint32_t n_tasks, int has_bias, int has_edges) {
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t task = xcd_remap(blockIdx.x, gridDim.x) * 4u + wave;
  if (task >= n_tasks) return;
  const uint32_t g = task / n_seg;
  const uint32_t seg = task - g * n_seg;
  const uint64_t *__restrict__ wg = words_in + (size_t)g * plane_stride;
  uint64_t *__restrict__ out = out_words + (size_t)g * out_stride;
  const uint32_t i0 = seg * 16u;

  const Key8 key = load_key(keys, g * 64u + lane);
  uint32_t x[16];
  chacha_block<8>(key.k, seg, x);

#pragma unroll 1
  for (int k = 0; k < 16; ++k) {
    const uint32_t i = i0 + k;
    if (i >= n_b) break;
    const uint32_t p = blk_off + i;
    float gam = 0.0f;
    if (has_bias) gam = gam + bias_w[p];
    if (has_edges) {
      const uint32_t a = row_off[p], b = row_off[p + 1];
      float acc = 0.0f;
      for (uint32_t s = a; s < b; ++s) {
        const uint2 sl = slots[s];
        const float wt = __builtin_bit_cast(float, sl.y);
        const uint64_t nw = wg[sl.x];
        const float sgn = lane_bit(nw) ? 1.0f : -1.0f;
        acc = (s == a) ? sgn * wt : f_fma(sgn, wt, acc);
      }
      gam = gam + acc;
    }
    const float prob = sigmoid_b(gam * 2.0f);
    uint32_t xk = x[0];
#pragma unroll
    for (int t = 1; t < 16; ++t) xk = (k == t) ? x[t] : xk;
    const uint64_t m = __builtin_amdgcn_ballot_w64(spin_uniform(xk) <= prob);
    if (lane == 0) out[i] = m;
  }
}

// ---------------------------------------------------------------------------
static inline uint32_t ceil_div(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

int launch_lattice_half(thrml_prog *p, thrml_state *st, uint32_t b, const uint32_t *d_keys) {
  const uint32_t ob = 1u - b;
  const uint32_t n_b = (uint32_t)(p->blk_off[b + 1] - p->blk_off[b]);
  const uint32_t n_seg = ceil_div(n_b, 16);
  const uint32_t n_tasks = n_seg * st->G;
  const uint32_t n_wg = ceil_div(n_tasks, 4);
  uint64_t *w = st->words.as<uint64_t>();
  const uint32_t *tab = p->table.as<uint32_t>() + (size_t)p->blk_off[b] * 16u;
  hipEvent_t t0 = nullptr;
  if (p->ctx->time_begin(0, &t0)) return THRML_EHIP;
  hipLaunchKernelGGL(lattice_half_kernel, dim3(n_wg), dim3(256), 0, p->ctx->stream,
                     w + p->blk_off[ob], w + p->blk_off[b], tab, d_keys, n_b, p->L, p->half,
                     p->parity[b], (uint64_t)p->n_total, n_seg, n_tasks);
  THRML_HIP(hipGetLastError());
  return p->ctx->time_end(0, t0);
}

int launch_csr_half(thrml_prog *p, thrml_state *st, uint32_t b, const uint32_t *d_keys) {
  const uint32_t n_b = (uint32_t)(p->blk_off[b + 1] - p->blk_off[b]);
  const uint32_t n_seg = ceil_div(n_b, 16);
  const uint32_t n_tasks = n_seg * st->G;
  const uint32_t n_wg = ceil_div(n_tasks, 4);
  uint64_t *w = st->words.as<uint64_t>();
  // With edges inside the block the new words go to a staging buffer first:
  // the block's new state replaces the old one only after the whole block
  // (crates/thrml-samplers/src/sampling.rs:57-59).
  uint64_t *dst = p->intra_block_edges ? st->scratch.as<uint64_t>() : w + p->blk_off[b];
  const uint64_t out_stride = p->intra_block_edges ? (uint64_t)n_b : p->n_total;
  const int has_bias = p->bias_raw.empty() ? 0 : 1;
  const int has_edges = p->eu.empty() ? 0 : 1;
  hipEvent_t t0 = nullptr;
  if (p->ctx->time_begin(0, &t0)) return THRML_EHIP;
  hipLaunchKernelGGL(csr_half_kernel, dim3(n_wg), dim3(256), 0, p->ctx->stream, w, dst,
                     p->row_off.as<uint32_t>(), p->slots.as<uint2>(), p->bias_w.as<float>(),
                     d_keys, n_b, (uint32_t)p->blk_off[b], (uint64_t)p->n_total, out_stride, n_seg,
                     n_tasks, has_bias, has_edges);
  THRML_HIP(hipGetLastError());
  if (int rc = p->ctx->time_end(0, t0)) return rc;
  if (p->intra_block_edges) {
    THRML_HIP(hipMemcpy2DAsync(w + p->blk_off[b], p->n_total * 8, dst, (size_t)n_b * 8,
                               (size_t)n_b * 8, st->G, hipMemcpyDeviceToDevice, p->ctx->stream));
  }
  return THRML_OK;
}

int launch_lattice_table(thrml_prog *p, const uint32_t *d_dir, const float *d_w,
                         const float *d_bias) {
  const uint32_t n = (uint32_t)p->blk_off[p->n_free];
  const uint32_t total = n * 16u;
  hipLaunchKernelGGL(lattice_table_kernel, dim3(ceil_div(total, 256)), dim3(256), 0,
                     p->ctx->stream, p->row_off.as<uint32_t>(), d_dir, d_w, d_bias, n,
                     p->bias_raw.empty() ? 0 : 1, p->eu.empty() ? 0 : 1, p->table.as<uint32_t>());
  THRML_HIP(hipGetLastError());
  return THRML_OK;
}

}  // namespace thrml
