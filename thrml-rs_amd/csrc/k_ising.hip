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
#include "dev_util.hpp"
#include "internal.hpp"

namespace thrml {

// ---------------------------------------------------------------------------
// Lattice half-sweep of block b on the L x L torus (L a multiple of 32).
//
// Block-local site i = r*half + t (half = L/2) sits in row r, column
// j = 2t + p with p = (r + par_b) & 1.  Its neighbours are words of the other
// block: in row r the words t + p - 1 (left, column j-1) and t + p (right,
// column j+1), taken modulo half; in rows r-1 and r+1 the word t (same
// column).  A wave takes 16 consecutive sites t0..t0+15 of one row (half is
// a multiple of 16), so its 49 neighbour words are three contiguous runs
// read with wide scalar loads.
//
// table[i][cfg] is the keystream-word threshold of site i for neighbour
// configuration cfg = L | R<<1 | U<<2 | D<<3 (1 = spin up); it was built with
// gamma summed in the reference's slot order, so `word <= table` is exactly
// `u <= sigmoid(2*gamma)`.  The configuration is formed directly as the byte
// offset 4*cfg into the site's 64-byte table row.
//
// Observed sweeps (mom != nullptr) also add the observation's moment counts:
// ones[pos] += #chains up at the updated sites, and for block 1 (updated
// last, when block 0 is final) diff[i*4 + d] += #chains whose spin differs
// from neighbour d.
struct LatticeArgs {
  const uint64_t *other;  // first word of the other block, group 0
  uint64_t *mine;         // first word of this block, group 0
  const uint32_t *table;  // this block's threshold rows
  const uint32_t *keys;   // [G*64][8] stream keys of this (sweep, block)
  uint32_t *ones;         // this block's node counters (observed sweeps) or null
  uint32_t *diff;         // block-1 edge counters or null
  uint64_t plane_stride;  // words per chain group
  uint32_t L, half, par, segs_row, n_seg, n_tasks, C;
};


__global__ __launch_bounds__(256) void lattice_half_kernel(LatticeArgs a) {
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t task = xcd_remap(blockIdx.x, gridDim.x) * 4u + wave;
  if (task >= a.n_tasks) return;
  const uint32_t g = task / a.n_seg;
  const uint32_t seg = task - g * a.n_seg;
  const uint32_t r = seg / a.segs_row;
  const uint32_t t0 = (seg - r * a.segs_row) * 16u;
  const uint32_t p = (r + a.par) & 1u;
  const uint32_t half = a.half;
  const uint64_t *oth = a.other + (size_t)g * a.plane_stride;
  const uint64_t *row = oth + (size_t)r * half;
  const uint64_t *up = oth + (size_t)(r == 0u ? a.L - 1u : r - 1u) * half + t0;
  const uint64_t *dn = oth + (size_t)(r + 1u == a.L ? 0u : r + 1u) * half + t0;
  const uint32_t lft0 = (t0 + p == 0u) ? half - 1u : t0 + p - 1u;   // left of site 0
  const uint32_t rgt15 = (t0 + p + 15u == half) ? 0u : t0 + p + 15u; // right of site 15
  const uint32_t i0 = r * half + t0;
  // the 16 table rows of this segment (1 KiB) as a buffer: 32-bit lane
  // offsets, row k at immediate offset 64k
  const __amdgpu_buffer_rsrc_t tab = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(a.table + (size_t)i0 * 16u), (short)0, 1024, 0x00020000);

  // thresholds: this lane's neighbour bits -> byte offset into the row
  uint32_t thr[16];
  {
    uint64_t lft = row[lft0];
    static_for<16>([&](auto k) {
      const uint64_t rgt = (k == 15) ? row[rgt15] : row[t0 + p + k];
      const uint32_t off = (lane_bit(lft) ? 4u : 0u) | (lane_bit(rgt) ? 8u : 0u) |
                           (lane_bit(up[k]) ? 16u : 0u) | (lane_bit(dn[k]) ? 32u : 0u);
      thr[k] = __builtin_amdgcn_raw_buffer_load_b32(tab, off, 64u * k, 0);
      lft = rgt;
    });
  }

  // this lane's 16 uniforms: keystream block i0/16 of the chain's key
  const Key8 key = load_key(a.keys, g * 64u + lane);
  uint32_t x[16];
  chacha_block<8>(key.k, i0 >> 4, x);

  const uint32_t live = a.C - g * 64u;
  const uint64_t valid = live >= 64u ? ~0ull : ((1ull << live) - 1ull);
  uint64_t m[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) m[k] = __builtin_amdgcn_ballot_w64(x[k] <= thr[k]) & valid;

  // edge counts of an observed block-1 update, before any store so that the
  // neighbour words are reloaded through the scalar cache (popcounts in SALU)
  uint32_t pk = 0u;
  if (a.diff) {
    const uint32_t z = opaque(0u);
    uint64_t lft = row[lft0 + z];
    static_for<16>([&](auto k) {
      const uint64_t rgt = (k == 15) ? row[rgt15 + z] : row[t0 + p + k + z];
      const uint32_t v = (uint32_t)__builtin_popcountll(m[k] ^ lft) |
                         ((uint32_t)__builtin_popcountll(m[k] ^ rgt) << 8) |
                         ((uint32_t)__builtin_popcountll(m[k] ^ up[k + z]) << 16) |
                         ((uint32_t)__builtin_popcountll(m[k] ^ dn[k + z]) << 24);
      pk = writelane<k>(pk, __builtin_amdgcn_readfirstlane(v));
      lft = rgt;
    });
  }

  // lanes 0..15 store the new words of sites 0..15
  uint32_t lo = 0u, hi = 0u;
  static_for<16>([&](auto k) {
    lo = writelane<k>(lo, (uint32_t)m[k]);
    hi = writelane<k>(hi, (uint32_t)(m[k] >> 32));
  });
  if (lane < 16u) {
    a.mine[(size_t)g * a.plane_stride + i0 + lane] = ((uint64_t)hi << 32) | lo;
    if (a.ones) atomicAdd(a.ones + i0 + lane, (uint32_t)(__builtin_popcount(lo) + __builtin_popcount(hi)));
    if (a.diff) {
      uint32_t *d = a.diff + (size_t)(i0 + lane) * 4u;
      atomicAdd(d + 0, pk & 0xffu);
      atomicAdd(d + 1, (pk >> 8) & 0xffu);
      atomicAdd(d + 2, (pk >> 16) & 0xffu);
      atomicAdd(d + 3, pk >> 24);
    }
  }
}

// Moment counts of one observation of a lattice state without a sweep (an
// observation that no sweep precedes): the same counters as the fused path.
// One thread per global position, summing over chain groups.
__global__ void lattice_moments_kernel(const uint64_t *__restrict__ words, uint64_t plane_stride,
                                       uint32_t G, uint32_t L, uint32_t half, uint32_t par1,
                                       uint32_t n_b, uint32_t *__restrict__ ones,
                                       uint32_t *__restrict__ diff) {
  const uint32_t pos = blockIdx.x * blockDim.x + threadIdx.x;
  if (pos >= 2u * n_b) return;
  uint32_t s = 0u;
  for (uint32_t g = 0; g < G; ++g) s += (uint32_t)__builtin_popcountll(words[(size_t)g * plane_stride + pos]);
  ones[pos] += s;
  if (pos < n_b) return;
  const uint32_t i = pos - n_b;
  const uint32_t r = i / half, t = i - r * half;
  const uint32_t p = (r + par1) & 1u;
  const uint32_t nb[4] = {r * half + (t + p == 0u ? half - 1u : t + p - 1u),
                          r * half + (t + p == half ? 0u : t + p),
                          (r == 0u ? L - 1u : r - 1u) * half + t,
                          (r + 1u == L ? 0u : r + 1u) * half + t};
  for (int d = 0; d < 4; ++d) {
    uint32_t c = 0u;
    for (uint32_t g = 0; g < G; ++g) {
      const uint64_t *w = words + (size_t)g * plane_stride;
      c += (uint32_t)__builtin_popcountll(w[pos] ^ w[nb[d]]);
    }
    diff[(size_t)i * 4u + d] += c;
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
    uint32_t n_tasks, int has_bias, int has_edges, uint32_t C) {
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
  const uint32_t live = C - g * 64u;
  const uint64_t valid = live >= 64u ? ~0ull : ((1ull << live) - 1ull);

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
    uint32_t xk = x[0];
#pragma unroll
    for (int t = 1; t < 16; ++t) xk = (k == t) ? x[t] : xk;
    const uint64_t m = __builtin_amdgcn_ballot_w64(spin_decision(gam * 2.0f, xk)) & valid;
    if (lane == 0) out[i] = m;
  }
}

// ---------------------------------------------------------------------------
static inline uint32_t ceil_div(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

int launch_lattice_half(thrml_prog *p, thrml_state *st, uint32_t b, const uint32_t *d_keys,
                        const LatticeMoments *mom) {
  const uint32_t ob = 1u - b;
  const uint32_t n_b = (uint32_t)(p->blk_off[b + 1] - p->blk_off[b]);
  if (p->half % 16u != 0u || (uint64_t)p->half * p->L != n_b)
    return fail(THRML_EINVAL, "lattice program with an unsupported shape");
  LatticeArgs a;
  uint64_t *w = st->words.as<uint64_t>();
  a.other = w + p->blk_off[ob];
  a.mine = w + p->blk_off[b];
  a.table = p->table.as<uint32_t>() + (size_t)p->blk_off[b] * 16u;
  a.keys = d_keys;
  a.ones = mom ? mom->ones + p->blk_off[b] : nullptr;
  a.diff = (mom && b == 1u) ? mom->diff : nullptr;
  a.plane_stride = p->n_total;
  a.L = p->L;
  a.half = p->half;
  a.par = p->parity[b];
  a.segs_row = p->half / 16u;
  a.n_seg = n_b / 16u;
  a.n_tasks = a.n_seg * st->G;
  a.C = st->C;
  const uint32_t n_wg = ceil_div(a.n_tasks, 4);
  hipEvent_t t0 = nullptr;
  if (p->ctx->time_begin(0, &t0)) return THRML_EHIP;
  hipLaunchKernelGGL(lattice_half_kernel, dim3(n_wg), dim3(256), 0, p->ctx->stream, a);
  THRML_HIP(hipGetLastError());
  return p->ctx->time_end(0, t0);
}

int launch_lattice_moments(thrml_state *st, const LatticeMoments *mom) {
  thrml_prog *p = st->prog;
  const uint32_t n_b = p->L * p->half;
  hipEvent_t t0 = nullptr;
  if (p->ctx->time_begin(1, &t0)) return THRML_EHIP;
  hipLaunchKernelGGL(lattice_moments_kernel, dim3(ceil_div(2ull * n_b, 256)), dim3(256), 0,
                     p->ctx->stream, st->words.as<uint64_t>(), (uint64_t)p->n_total, st->G, p->L,
                     p->half, p->parity[1], n_b, mom->ones, mom->diff);
  THRML_HIP(hipGetLastError());
  return p->ctx->time_end(1, t0);
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
                     n_tasks, has_bias, has_edges, st->C);
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
