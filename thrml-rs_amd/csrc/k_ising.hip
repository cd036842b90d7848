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
#include <algorithm>

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
  const uint32_t *keys;   // [G*64][KEY_WORDS] stream keys of this (sweep, block)
  uint32_t *ones;         // this block's node counters (observed sweeps) or null
  uint32_t *diff;         // block-1 edge counters or null
  uint64_t plane_stride;  // words per chain group
  uint32_t L, half, par, segs_row, n_seg, n_tasks, C;
  uint32_t excl;          // one chain group: each counter has one writer per launch
  FastDiv div_seg, div_row;  // by n_seg, by segs_row
};


__global__ __launch_bounds__(256) void lattice_half_kernel(LatticeArgs a) {
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t task = xcd_remap(blockIdx.x, gridDim.x) * 4u + wave;
  if (task >= a.n_tasks) return;
  const uint32_t g = fdiv(task, a.div_seg);
  const uint32_t seg = task - g * a.n_seg;
  const uint32_t r = fdiv(seg, a.div_row);
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
  // the 16 table rows of this segment (1 KiB) go to this wave's LDS with one
  // coalesced 16-byte load per lane, issued together with the neighbour
  // loads (the global access no longer waits for the neighbour words); each
  // lane then reads its entry of row k at word 16k + cfg
  __shared__ uint32_t tabs[4][256];
  uint32_t *mytab = tabs[wave];
  reinterpret_cast<uint4 *>(mytab)[lane] =
      reinterpret_cast<const uint4 *>(a.table + (size_t)i0 * 16u)[lane];

  // thresholds: this lane's neighbour bits -> LDS address of the entry
  uint32_t thr[16];
  {
    // a site's left neighbour is the previous site's right one: each word's
    // bit is materialised once as 0 / 4 and doubled where it is a right bit
    // (one v_lshl_or_b32).  The down bit selects between the row base and
    // base + 32, both held in registers, so the address is complete after
    // one more v_or3_b32: five instructions per site.
    const uint32_t base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)mytab;
    const uint32_t b0 = opaque(base), b32 = opaque(base + 32u);
    uint32_t l4 = lane_bit(row[lft0]) ? 4u : 0u;
    static_for<16>([&](auto k) {
      const uint64_t rgt = (k == 15) ? row[rgt15] : row[t0 + p + k];
      const uint32_t r4 = lane_bit(rgt) ? 4u : 0u;
      const uint32_t u16 = lane_bit(up[k]) ? 16u : 0u;
      const uint32_t db = lane_bit(dn[k]) ? b32 : b0;
      uint32_t lr;
      asm("v_lshl_or_b32 %0, %1, 1, %2" : "=v"(lr) : "v"(r4), "v"(l4));
      const uint32_t addr = lr | u16 | db;
      thr[k] = *reinterpret_cast<const __attribute__((address_space(3))) uint32_t *>(
          (uintptr_t)(addr + 64u * k));
      l4 = r4;
    });
  }

  // this lane's 16 uniforms: keystream block i0/16 of the chain's key
  uint32_t key[KEY_WORDS];
  load_keyx(a.keys, g * 64u + lane, key);
  uint32_t x[16];
  chacha_block_pre<8>(key, i0 >> 4, x);

  const uint32_t live = a.C - g * 64u;
  const uint64_t valid = live >= 64u ? ~0ull : ((1ull << live) - 1ull);
  uint64_t m[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) m[k] = __builtin_amdgcn_ballot_w64(x[k] <= thr[k]) & valid;

  // lanes 0..15 store the new words of sites 0..15
  uint32_t lo = 0u, hi = 0u;
  static_for<16>([&](auto k) {
    lo = writelane<k>(lo, (uint32_t)m[k]);
    hi = writelane<k>(hi, (uint32_t)(m[k] >> 32));
  });
  if (lane < 16u) {
    a.mine[(size_t)g * a.plane_stride + i0 + lane] = ((uint64_t)hi << 32) | lo;
    const uint32_t pop = (uint32_t)(__builtin_popcount(lo) + __builtin_popcount(hi));
    // edge counts of an observed block-1 update: lane k takes site k and its
    // four neighbour words (the other block, unchanged by this launch)
    uint4 dv = make_uint4(0u, 0u, 0u, 0u);
    if (a.diff) {
      const uint32_t li = t0 + p + lane;
      const uint64_t nb[4] = {row[lane == 0u ? lft0 : li - 1u], row[lane == 15u ? rgt15 : li],
                              up[lane], dn[lane]};
      uint32_t c[4];
#pragma unroll
      for (int d = 0; d < 4; ++d)
        c[d] = (uint32_t)(__builtin_popcount(lo ^ (uint32_t)nb[d]) +
                          __builtin_popcount(hi ^ (uint32_t)(nb[d] >> 32)));
      dv = make_uint4(c[0], c[1], c[2], c[3]);
    }
    if (a.excl) {
      // the only writer of these counters in this launch: plain read-modify-write
      if (a.ones) a.ones[i0 + lane] += pop;
      if (a.diff) {
        uint4 *d4 = reinterpret_cast<uint4 *>(a.diff) + i0 + lane;
        uint4 v = *d4;
        v.x += dv.x;
        v.y += dv.y;
        v.z += dv.z;
        v.w += dv.w;
        *d4 = v;
      }
    } else {
      if (a.ones) atomicAdd(a.ones + i0 + lane, pop);
      if (a.diff) {
        uint32_t *d = a.diff + (size_t)(i0 + lane) * 4u;
        atomicAdd(d + 0, dv.x);
        atomicAdd(d + 1, dv.y);
        atomicAdd(d + 2, dv.z);
        atomicAdd(d + 3, dv.w);
      }
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
// that order, acc = fl(acc + (+-w)) from 0, then gamma = (0 + bias) + acc.
//
// A wave takes a run of RUN consecutive sites of 64 chains (FULL), or, with
// at most 32 chains (HALF), two runs side by side (lanes 32..63 take the
// second), so that no lane idles.  RUN is 16 (one ChaCha8 block of uniforms
// per lane) or, for blocks too small to fill the GPU, 4 (a quarter of a
// block: shorter serial work per wave, more waves).  HALF always takes 4-site
// runs: the workgroup's four waves then cover 32 consecutive sites, two
// keystream blocks per chain, which wave 0 computes (one block per lane)
// into LDS for all four, so that no keystream word is computed and thrown
// away.  The keystream is computed while the neighbour words are in flight.
// The slot records of a
// wave's sites are contiguous: the wave gathers them and their neighbours'
// state words in one round trip each and stages each slot in LDS as
// {sign mask, |w|}, where bit c of the sign mask is set iff the slot's
// contribution for chain c is negative, so that a contribution is one shift
// and one bit-field insert.  Each lane then walks its site's slots four at a
// time (two paired 64-bit LDS reads); in HALF mode the two runs' sites differ
// in length, so the groups past the shorter one are masked (weight 0).  The
// LDS stage per wave is sized by the launch for the block's largest window;
// a wave whose slots exceed the largest stage reads them from global memory
// in the same order instead.
constexpr uint32_t STAGE_MAX_U2 = 2048;  // uint2 entries per wave at most (16 KiB, padding included)
constexpr uint32_t STAGE_PAD_U2 = 8;     // read-ahead room past the last slot

struct CsrArgs {
  const uint64_t *words;   // state words, group 0
  uint64_t *out;           // new words of this block, group 0
  // HALF (at most 32 chains): neighbour states are the u32 low[pos << low_shift]
  // (the state's low-half copy with shift 0, else the words' low halves
  // with shift 1); out_low, when set, takes this block's new low halves
  const uint32_t *low;
  uint32_t *out_low;
  uint32_t low_shift;
  const uint32_t *row_off; // [n_free + 1]
  const uint2 *slots;      // padded by 16 zero records
  const float *bias_w;     // [n_free] fl(beta * b)
  const uint32_t *keys;
  uint64_t plane_stride, out_stride;
  uint32_t n_b, blk_off, n_seg, n_tasks, has_bias, has_edges, C;
  uint32_t stage_u2;       // LDS entries per wave (>= STAGE_PAD_U2)
  FastDiv div_seg;         // by n_seg
};

// {sign mask, |w|} of slot record `r` for the chains in word half `hi`
__device__ __forceinline__ uint2 slot_entry(uint2 r, uint64_t nw, bool hi) {
  const uint32_t d = hi ? (uint32_t)(nw >> 32) : (uint32_t)nw;
  // contribution = bit ? w : -w, negative iff bit == sign(w)
  const uint32_t m = (r.y & 0x80000000u) ? d : ~d;
  return make_uint2(m, r.y & 0x7fffffffu);
}

// signed contribution of staged slot `e` for the chain at bit `sh`
__device__ __forceinline__ float slot_value(uint2 e, uint32_t sh, uint32_t mag) {
  return __builtin_bit_cast(float, ((e.x << (31u - sh)) & 0x80000000u) | mag);
}

// PM > 0: every site of the block has at most 8 PM slots, so every wave
// takes the per-site regions (copied in PM passes) and the kernel carries no
// other staging path (fewer registers: eight waves per SIMD, not seven).
template <bool HALF, int RUN, int PM>
__global__ __launch_bounds__(256) void csr_half_kernel(CsrArgs a) {
  constexpr int NIT = PM ? PM : 4;  // region copy passes of 8 slots
  constexpr uint32_t PER = HALF ? 1u : 2u;            // LDS entries per slot
  constexpr uint32_t SITES = HALF ? 2u * RUN : RUN;   // sites per wave
  extern __shared__ uint2 stage_all[];
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  uint2 *stage = stage_all + wave * a.stage_u2;
  const uint32_t cap = (a.stage_u2 - STAGE_PAD_U2) / PER;  // slots a stage holds
  // HALF, RUN 4: the workgroup's 32 sites take two keystream blocks per
  // chain; wave 0 computes them (lane = chain + 32 * block) into LDS
  constexpr bool SHARE = HALF && RUN == 4;
  uint32_t *ks = reinterpret_cast<uint32_t *>(stage_all + 4u * a.stage_u2);
  const uint32_t wg0 = xcd_remap(blockIdx.x, gridDim.x);
  const uint32_t task = wg0 * 4u + wave;
  const bool active = task < a.n_tasks;  // (no early return: the waves share a barrier)
  // a wave past the last task takes task 0's addresses (its chain group and
  // records exist) and writes nothing: with task itself its group index could
  // be G, one plane past the state words, which its staging loads would read
  const uint32_t tsk = active ? task : 0u;
  const uint32_t g = HALF ? 0u : fdiv(tsk, a.div_seg);
  const uint32_t segA = HALF ? tsk * 2u : tsk - g * a.n_seg;
  const uint32_t h = HALF ? lane >> 5 : 0u;  // run of this lane
  const uint32_t chain = HALF ? (lane & 31u) : g * 64u + lane;
  const uint32_t i0w = segA * RUN;
  const uint32_t rs = i0w + RUN * h;         // first site of this lane's run
  const uint32_t iend = active ? min(a.n_b, i0w + SITES) : i0w;
  const bool lane_ok = active && rs < iend && chain < a.C;
  const uint64_t *__restrict__ wg = a.words + (size_t)g * a.plane_stride;
  // neighbour state word at global position `pos` (HALF reads only its low half)
  auto nbr = [&](uint32_t pos) -> uint64_t {
    if constexpr (HALF) return a.low[(size_t)pos << a.low_shift];
    else return wg[pos];
  };
  const uint32_t sh = lane & 31u;
  const uint32_t half_off = HALF ? 0u : (lane >> 5);  // which LDS entry of a slot this lane reads
  const bool hi_word = !HALF && lane >= 32u;

  // per-site row offsets and biases of the wave: lane l holds site i0w + l
  const uint32_t lrow = min(i0w + lane, iend);
  uint32_t ro = 0u;
  float bl = 0.0f;
  if (active && a.has_edges && lane <= SITES) ro = a.row_off[a.blk_off + lrow];
  if (active && a.has_bias && lrow < iend) bl = a.bias_w[a.blk_off + lrow];
  uint32_t key[KEY_WORDS];
#pragma unroll
  for (int i = 0; i < KEY_WORDS; ++i) key[i] = 0u;
  if (SHARE) {
    if (wave == 0u && chain < a.C) load_keyx(a.keys, chain, key);
  } else if (lane_ok) {
    load_keyx(a.keys, chain, key);
  }
  const uint32_t r0 = __builtin_amdgcn_readfirstlane(ro);
  const uint32_t T = __builtin_amdgcn_readlane(ro, iend - i0w) - r0;
  // HALF: the wave's 9 site offsets in scalar registers, and the largest
  // site degree md.  With md <= 8 NIT each site takes a region of P = md
  // rounded up to 4 entries, whose entries past the site's degree have magnitude 0,
  // so that both runs' sums run to the longer site without masks (a zero
  // contribution is exact: the running sum starts at +0 and is never -0).
  uint32_t so[HALF ? 9 : 1];
  uint32_t md = 0u;
  if constexpr (HALF) {
#pragma unroll
    for (int q = 0; q < 9; ++q) so[q] = __builtin_amdgcn_readlane(ro, q);
#pragma unroll
    for (int q = 0; q < 8; ++q) md = max(md, so[q + 1] - so[q]);
  }
  const uint32_t P = (md + 3u) & ~3u;
  const bool pmode = HALF && (PM || (md <= 8u * NIT && 8u * P <= cap));
  const bool staged = pmode || T <= cap;
  uint32_t x[16] = {};
  const uint32_t tl = T ? T - 1u : 0u;  // the wave's last record
  // pmode: lanes 8s..8s+7 copy site s's slots lt, lt + 8, lt + 16, ...
  // into its region (reads past the degree are clamped to its last record
  // and stored with magnitude 0).  Otherwise the first 512 slots of the
  // wave's records go to consecutive entries without a branch (clamped reads
  // stay inside the wave's records, or on the padding record when it has
  // none), and the rest, if any, in a loop.
  const uint32_t ls = lane >> 3, lt = lane & 7u;
  uint32_t dsite = 0u;
  uint2 rec[8];
  if (pmode) {
    const uint32_t rsite = __shfl(ro, (int)ls);
    dsite = __shfl(ro, (int)ls + 1) - rsite;
    const uint32_t dlast = dsite ? dsite - 1u : 0u;
#pragma unroll
    for (uint32_t q = 0; q < NIT; ++q) rec[q] = a.slots[rsite + min(lt + 8u * q, dlast)];
  } else if constexpr (!PM) {
#pragma unroll
    for (uint32_t q = 0; q < 8; ++q) rec[q] = a.slots[r0 + min(q * 64u + lane, tl)];
  }
  if (!SHARE || wave == 0u) chacha_block_pre<8>(key, SHARE ? 2u * wg0 + h : rs >> 4, x);
  // SHARE: wave 0 publishes the keystream words as soon as they exist (its
  // registers are then free for the staging)
  auto publish = [&]() {
    if constexpr (SHARE) {
      if (wave == 0u) {
#pragma unroll
        for (int i = 0; i < 16; ++i) ks[i * 64 + lane] = x[i];
      }
    }
  };
  if (pmode) {
    uint64_t nw[NIT];
#pragma unroll
    for (uint32_t q = 0; q < NIT; ++q) nw[q] = nbr(rec[q].x);
    // the keystream block while the neighbour words are in flight
#pragma unroll
    for (int i = 0; i < 16; ++i) asm volatile("" : "+v"(x[i]));
    publish();
    // entry lt + 8q of the region; rem = this lane's slots from lt on
    uint2 *const dst = stage + ls * P + lt;
    const int32_t rem = (int32_t)dsite - (int32_t)lt;
#pragma unroll
    for (uint32_t q = 0; q < NIT; ++q) {
      uint2 e = slot_entry(rec[q], nw[q], false);
      e.y = rem > (int32_t)(8u * q) ? e.y : 0u;
      if ((int32_t)lt < (int32_t)P - (int32_t)(8u * q)) dst[8u * q] = e;
    }
  } else if (!PM && staged) {
    uint64_t nw[8];
#pragma unroll
    for (uint32_t q = 0; q < 8; ++q) nw[q] = nbr(rec[q].x);
    // the keystream block while the neighbour words are in flight
#pragma unroll
    for (int i = 0; i < 16; ++i) asm volatile("" : "+v"(x[i]));
    publish();
#pragma unroll
    for (uint32_t q = 0; q < 8; ++q) {
      const uint32_t idx = q * 64u + lane;
      if (idx < T) {
        stage[idx * PER] = slot_entry(rec[q], nw[q], false);
        if (!HALF) stage[idx * PER + 1] = slot_entry(rec[q], nw[q], true);
      }
    }
    // (256 records per pass: fewer registers than the first pass's 512)
    for (uint32_t base = 512u; base < T; base += 256u) {
#pragma unroll
      for (uint32_t q = 0; q < 4; ++q) rec[q] = a.slots[r0 + min(base + q * 64u + lane, tl)];
#pragma unroll
      for (uint32_t q = 0; q < 4; ++q) nw[q] = nbr(rec[q].x);
#pragma unroll
      for (uint32_t q = 0; q < 4; ++q) {
        const uint32_t idx = base + q * 64u + lane;
        if (idx < T) {
          stage[idx * PER] = slot_entry(rec[q], nw[q], false);
          if (!HALF) stage[idx * PER + 1] = slot_entry(rec[q], nw[q], true);
        }
      }
    }
  } else {
    publish();
  }
  if constexpr (SHARE) {
    __syncthreads();
  } else {
    // each wave reads only its own staging region: a wavefront-scope fence
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // SHARE: site 4h + k of wave w takes keystream word lw = 8w + 4h + k, at
  // ks[(lw & 15) * 64 + chain + 32 (lw >> 4)]: the lane's four words are 64
  // apart from one base, computed once (the asm keeps the compiler from
  // recomputing it per site)
  const uint32_t *ksp = ks;
  if constexpr (SHARE) {
    const uint32_t lw0 = 8u * wave + 4u * h;
    uint32_t o = (lw0 & 15u) * 64u + (lane & 31u) + 32u * (lw0 >> 4);
    asm("" : "+v"(o));
    ksp = ks + o;
  }
  uint32_t wa = 0u, wb = 0u;  // new words of lanes 0..RUN-1: run 0 / run 1 (HALF), lo / hi (FULL)
  static_for<RUN>([&](auto k_c) {
    constexpr int k = decltype(k_c)::value;
    // slot ranges of this lane's site (run 0 site: lane k of ro; run 1: lane RUN + k)
    uint32_t a0, a1;
    if constexpr (HALF) {
      a0 = so[k];
      a1 = so[k + 1];
    } else {
      a0 = __builtin_amdgcn_readlane(ro, k);
      a1 = __builtin_amdgcn_readlane(ro, k + 1);
    }
    uint32_t s_beg = a0, deg = a1 - a0, trips = deg, common = deg;
    float bias = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(uint32_t, bl), k));
    if constexpr (HALF) {
      const uint32_t b0 = so[RUN + k];
      const uint32_t b1 = so[RUN + k + 1];
      trips = max(deg, b1 - b0);
      common = min(deg, b1 - b0);
      const float bb = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(uint32_t, bl), RUN + k));
      if (h) {
        s_beg = b0;
        deg = b1 - b0;
        bias = bb;
      }
    }
    float acc = 0.0f;
    if (a.has_edges) {
      const uint32_t rel = s_beg - r0;
      uint32_t t = 0;
      if (pmode) {
        // this lane's site region: sums to the longer site of the pair, unmasked
        const uint2 *sp = stage + ((uint32_t)k + RUN * h) * P;
        for (; t < trips; t += 4u) {
          uint2 e[4];
#pragma unroll
          for (uint32_t u = 0; u < 4; ++u) e[u] = sp[t + u];
#pragma unroll
          for (uint32_t u = 0; u < 4; ++u) acc = acc + slot_value(e[u], sh, e[u].y);
        }
      } else if (!PM && staged) {
        // groups every lane's site fills: no mask
        for (; t + 4u <= common; t += 4u) {
          const uint2 *sp = stage + (rel + t) * PER + half_off;
          uint2 e[4];
#pragma unroll
          for (uint32_t u = 0; u < 4; ++u) e[u] = sp[u * PER];
#pragma unroll
          for (uint32_t u = 0; u < 4; ++u) acc = acc + slot_value(e[u], sh, e[u].y);
        }
        if constexpr (HALF) {
          for (; t < trips; t += 4u) {
            const uint2 *sp = stage + min(rel + t, cap) * PER + half_off;
            uint2 e[4];
#pragma unroll
            for (uint32_t u = 0; u < 4; ++u) e[u] = sp[u * PER];
#pragma unroll
            for (uint32_t u = 0; u < 4; ++u) acc = acc + slot_value(e[u], sh, t + u < deg ? e[u].y : 0u);
          }
        } else {
          // FULL: every lane sums the same site, so its last slots are a
          // wave-uniform loop instead of a masked group
          for (; t < deg; ++t) {
            const uint2 e = stage[(rel + t) * PER + half_off];
            acc = acc + slot_value(e, sh, e.y);
          }
        }
      } else {
        for (; t < trips; t += 4u) {
          uint2 r[4];
#pragma unroll
          for (uint32_t u = 0; u < 4; ++u) r[u] = a.slots[min(s_beg + t + u, r0 + tl)];
          uint2 e[4];
#pragma unroll
          for (uint32_t u = 0; u < 4; ++u) e[u] = slot_entry(r[u], nbr(r[u].x), hi_word);
#pragma unroll
          for (uint32_t u = 0; u < 4; ++u) acc = acc + slot_value(e[u], sh, t + u < deg ? e[u].y : 0u);
        }
      }
    }
    float gam = 0.0f;
    if (a.has_bias) gam = gam + bias;
    gam = gam + acc;
    uint32_t xk;
    if constexpr (RUN == 16) {
      xk = x[k];
    } else if constexpr (SHARE) {
      xk = ksp[k * 64];
    } else {  // run start rs % 16 in {0, 4, 8, 12}: word rs % 16 + k
      const uint32_t qd = (rs >> 2) & 3u;
      const uint32_t lo = (qd & 1u) ? x[4 + k] : x[k];
      const uint32_t hi = (qd & 1u) ? x[12 + k] : x[8 + k];
      xk = (qd & 2u) ? hi : lo;
    }
    const bool up = lane_ok && (rs + k < iend) && spin_decision(gam, xk);
    const uint64_t m = __builtin_amdgcn_ballot_w64(up);
    wa = writelane<k>(wa, (uint32_t)m);
    wb = writelane<k>(wb, (uint32_t)(m >> 32));
  });
  if (active && lane < (uint32_t)RUN) {
    if (HALF) {
      if (i0w + lane < iend) a.out[i0w + lane] = wa;
      if (i0w + RUN + lane < iend) a.out[i0w + RUN + lane] = wb;
      if (a.out_low) {
        if (i0w + lane < iend) a.out_low[i0w + lane] = wa;
        if (i0w + RUN + lane < iend) a.out_low[i0w + RUN + lane] = wb;
      }
    } else if (i0w + lane < iend) {
      a.out[(size_t)g * a.out_stride + i0w + lane] = ((uint64_t)wb << 32) | wa;
    }
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
  a.excl = st->G == 1u ? 1u : 0u;
  a.segs_row = p->half / 16u;
  a.n_seg = n_b / 16u;
  a.div_seg = make_fastdiv(a.n_seg);
  a.div_row = make_fastdiv(a.segs_row);
  // task indices are divided by n_seg with a reciprocal exact below 2^31
  if ((uint64_t)a.n_seg * st->G >= (1ull << 31))
    return fail(THRML_EINVAL, "lattice block too large: segments x chain groups must stay below 2^31");
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

// Largest slot count of a wave's window of `w` sites (windows aligned at
// multiples of w) in each free block, for w = 4, 8, 16, 32, and the largest
// slot count of one site.
void csr_windows(thrml_prog *p, const std::vector<uint32_t> &row_off) {
  p->csr_maxdeg.assign(p->n_free, 0u);
  for (uint32_t b = 0; b < p->n_free; ++b)
    for (uint64_t i = p->blk_off[b]; i < p->blk_off[b + 1]; ++i)
      p->csr_maxdeg[b] = std::max(p->csr_maxdeg[b], row_off[i + 1] - row_off[i]);
  static const uint32_t ws[4] = {4, 8, 16, 32};
  for (int wi = 0; wi < 4; ++wi) {
    std::vector<uint32_t> &mx = p->csr_win[wi];
    mx.assign(p->n_free, 0u);
    for (uint32_t b = 0; b < p->n_free; ++b) {
      const uint64_t lo = p->blk_off[b], hi = p->blk_off[b + 1];
      for (uint64_t i = lo; i < hi; i += ws[wi]) {
        const uint64_t e = std::min<uint64_t>(i + ws[wi], hi);
        mx[b] = std::max(mx[b], row_off[e] - row_off[i]);
      }
    }
  }
}

template <bool HALF, int RUN, int PM = 0>
static void launch_csr_t(const CsrArgs &a, hipStream_t s) {
  hipLaunchKernelGGL((csr_half_kernel<HALF, RUN, PM>), dim3(ceil_div(a.n_tasks, 4)), dim3(256),
                     (size_t)4 * a.stage_u2 * sizeof(uint2) + (HALF && RUN == 4 ? 4096u : 0u), s, a);
}

int launch_csr_half(thrml_prog *p, thrml_state *st, uint32_t b, const uint32_t *d_keys) {
  const uint32_t n_b = (uint32_t)(p->blk_off[b + 1] - p->blk_off[b]);
  CsrArgs a;
  uint64_t *w = st->words.as<uint64_t>();
  a.words = w;
  // A staged block writes into the staging buffer: its new state replaces
  // the old one only after its superblock (crates/thrml-samplers/src/sampling.rs:39-60)
  uint64_t soff = 0, swidth = 0;
  if (stage_target(p, b, &soff, &swidth)) {
    a.out = st->scratch.as<uint64_t>() + soff;
    a.out_stride = swidth;
  } else {
    a.out = w + p->blk_off[b];
    a.out_stride = p->n_total;
  }
  // a state keeps its low-half copy only when no block is staged
  if (st->low.p) {
    a.low = st->low.as<uint32_t>();
    a.out_low = st->low.as<uint32_t>() + p->blk_off[b];
    a.low_shift = 0u;
  } else {
    a.low = reinterpret_cast<const uint32_t *>(w);
    a.out_low = nullptr;
    a.low_shift = 1u;
  }
  a.row_off = p->row_off.as<uint32_t>();
  a.slots = p->slots.as<uint2>();
  a.bias_w = p->bias_w.as<float>();
  a.keys = d_keys;
  a.plane_stride = p->n_total;
  a.n_b = n_b;
  a.blk_off = (uint32_t)p->blk_off[b];
  a.has_bias = p->bias_raw.empty() ? 0u : 1u;
  a.has_edges = p->eu.empty() ? 0u : 1u;
  a.C = st->C;
  const bool half = st->C <= 32u;
  // Up to 32 chains: 4-site runs, whose workgroup shares its keystream blocks
  // (config 3: 184 us per sweep against 201 us with 16-site runs on its four
  // largest blocks).  More chains: 16-site runs while they give at least 16
  // waves per CU, else 4-site runs (8 or 32 waves per CU as the limit are
  // 3-8 % slower).
  const uint32_t waves16 = ceil_div(n_b, 16) * st->G;
  const int run = !half && waves16 >= 4096u ? 16 : 4;
  a.n_seg = ceil_div(n_b, run);
  a.div_seg = make_fastdiv(a.n_seg);
  if ((uint64_t)a.n_seg * st->G >= (1ull << 31))
    return fail(THRML_EINVAL, "block too large: runs x chain groups must stay below 2^31");
  a.n_tasks = half ? ceil_div(a.n_seg, 2) : a.n_seg * st->G;
  // window of one wave: 2*run sites (HALF) or run sites (FULL)
  const uint32_t wsites = half ? 2u * run : (uint32_t)run;
  const int wi = wsites == 4 ? 0 : wsites == 8 ? 1 : wsites == 16 ? 2 : 3;
  const uint32_t per = half ? 1u : 2u;
  uint64_t want = (uint64_t)p->csr_win[wi][b] * per + STAGE_PAD_U2;
  // HALF: room for eight 4-aligned site regions of up to 40 slots each
  if (half) want = std::max<uint64_t>(want, 8u * ((std::min(p->csr_maxdeg[b], 40u) + 3u) & ~3u) + STAGE_PAD_U2);
  a.stage_u2 = (uint32_t)std::min<uint64_t>((want + 7u) & ~7ull, STAGE_MAX_U2);
  hipEvent_t t0 = nullptr;
  if (p->ctx->time_begin(0, &t0)) return THRML_EHIP;
  hipStream_t s = p->ctx->stream;
  if (half) {
    const uint32_t md = p->csr_maxdeg[b];
    if (md <= 32u) launch_csr_t<true, 4, 4>(a, s);
    else if (md <= 40u) launch_csr_t<true, 4, 5>(a, s);
    else launch_csr_t<true, 4>(a, s);
  }
  else
    run == 16 ? launch_csr_t<false, 16>(a, s) : launch_csr_t<false, 4>(a, s);
  THRML_HIP(hipGetLastError());
  return p->ctx->time_end(0, t0);
}

__global__ __launch_bounds__(256) void pack_low_kernel(const uint64_t *__restrict__ w,
                                                       uint32_t *__restrict__ low, uint64_t n) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    low[i] = (uint32_t)w[i];
}

int launch_pack_low(thrml_state *st) {
  thrml_prog *p = st->prog;
  const uint64_t n = p->n_total;
  if (n == 0) return THRML_OK;
  const uint32_t grid = (uint32_t)std::min<uint64_t>((n + 255u) / 256u, 8192u);
  hipLaunchKernelGGL(pack_low_kernel, dim3(grid), dim3(256), 0, p->ctx->stream,
                     st->words.as<uint64_t>(), st->low.as<uint32_t>(), n);
  THRML_HIP(hipGetLastError());
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
