// k_potts.hip -- categorical (Potts) half-sweep for gfx950.
//
// One launch updates one free block of every chain with
// CategoricalGibbsConditional (crates/thrml-samplers/src/softmax.rs:228-271):
//   theta[c] = ((0 + b[x][c]) + sum_{u-role slots} W[e][c][x_v])
//                             + sum_{v-role slots} W[e][x_u][c]
// (compute_parameters, softmax.rs:586-710, over the interaction groups of
// DiscreteEBMFactor::to_interaction_groups, crates/thrml-models/src/discrete_ebm.rs:456-548:
// bias group, head-U group with W, head-V group with W.swap_dims(1, 2)), each
// group summed over its slots in ascending order before it is added; then
// x' = first argmax_c(theta[c] - log(-log u_c)) (categorical_sample,
// softmax.rs:60-97; first maximum as gumbel_argmax/kernel.rs:81-83).
//
// State: one byte per (global position, chain), chains fastest
// ([n_total][Cp], Cp = C rounded up to 4).  Work decomposition: a lane takes
// one chain and a run of S = lcm(Q, 16) / Q consecutive block-local sites,
// whose Q * S keystream words (site i, category c -> word i*Q + c of the
// block key's ChaCha8 stream) are exactly lcm(Q, 16) / 16 whole ChaCha8
// blocks; lanes of one wave are consecutive chains of the same run, so a
// site's slot lists and bias row are shared by the wave and the chains'
// neighbour bytes are contiguous.  Q = 17..256 (potts_wide_kernel): a lane
// takes one site and walks its categories one keystream block at a time.
#include "dev_util.hpp"
#include "internal.hpp"

namespace thrml {

struct PottsArgs {
  const uint8_t *state;     // [n_total][Cp]
  uint8_t *out;             // new categories of this block: [n_b][Cp]
  const uint32_t *row_off;  // [nf + 1] first slot of each free position
  const uint32_t *uend;     // [nf] end of the position's u-role slots
  const uint2 *slots;       // {tail position, edge id}
  const uint4 *pslots;      // role-padded slots: [nf][M] uint4 = 2M {tail, edge} pairs
  const float *bias;        // [nf][Q] = 0 + b
  const float *W;           // [E+1][Q][Q] (edge E all zeros)
  const float *Wt;          // [E+1][Q][Q] transposes
  const uint32_t *keys;     // [G*64][KEY_WORDS] stream keys of this (sweep, block)
  uint32_t n_b, blk_off, C, Cp, n_items, has_edges;
  FastDiv div_c;            // by C
  uint32_t items_per_part;  // generic kernel: items of one sub-run part, a multiple of 64
  uint32_t n_edges;         // E: the id of the all-zero padding edge
  uint32_t narrow;          // potts_narrow holds
};

// The LDS-staged role-padded kernel addresses the state and the weight
// matrices with 32-bit offsets from their bases, and multiplies a tail
// position by Cp in 24 bits: it runs only when these fit.
static inline bool potts_narrow(uint64_t n_total, uint32_t Cp, uint64_t n_edges, uint32_t Q) {
  return n_total < (1ull << 24) && Cp < (1u << 24) && n_total * Cp < (1ull << 32) &&
         (n_edges + 1) * Q * Q * 4u <= (1ull << 32);
}

constexpr int gcd_c(int a, int b) { return b == 0 ? a : gcd_c(b, a % b); }

// potts_pick for a lane whose S sites take exactly one keystream block
// (lcm(Q, 16) = 16), with that block's 16 fast Gumbel scores computed ahead
// (gs[w] = gumbel_fast(word w)): the role-padded kernel computes them while
// its first site's slot records are in flight (config 4: 4 % less time per
// launch than computing the block at the first pick).
template <int Q>
__device__ __forceinline__ uint32_t potts_pick_pre(const float (&th)[Q], int s, const float (&gs)[16],
                                                   const uint32_t *keys, uint32_t c, uint64_t ctr0) {
  // first maximum and runner-up: with best >= second, the new runner-up is
  // the median of (v, best, second), and v replaces best only if greater
  float best = th[0] + gs[(s * Q) & 15], second = -INFINITY;
  uint32_t arg = 0;
#pragma unroll
  for (int q = 1; q < Q; ++q) {
    const float v = th[q] + gs[(s * Q + q) & 15];
    const bool gt = v > best;
    second = __builtin_amdgcn_fmed3f(v, best, second);
    arg = gt ? (uint32_t)q : arg;
    best = gt ? v : best;
  }
  if (!(best - second > gumbel_margin(best, second))) {
    uint32_t key[8], eb[16];
    load_key8(keys, c, key);
    chacha_block<8>(key, ctr0, eb);
    best = 0.0f;
    arg = 0;
    for (int q = 0; q < Q; ++q) {
      const int rel = s * Q + q;
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

// Sum of the weight rows of slots k0..k1-1 of one role, in slot order (0 for
// no slots).  U slots at a time: their records, then their tail bytes, then
// their rows are loaded together, so a site's chains of dependent loads
// (record -> tail byte -> row) overlap U-fold; the slots past k1 of the last
// group load slot k1 - 1 again and add nothing.
template <int Q, int U>
__device__ __forceinline__ void role_rows(const PottsArgs &a, uint32_t c, uint32_t k0, uint32_t k1,
                                          const float *w, float (&sr)[Q]) {
#pragma unroll
  for (int q = 0; q < Q; ++q) sr[q] = 0.0f;
  if constexpr (U == 1) {
    for (uint32_t k = k0; k < k1; ++k) {
      const uint2 sl = a.slots[k];
      const uint32_t xt = a.state[(size_t)sl.x * a.Cp + c];
      float we[Q];
      load_row<Q>(w + ((size_t)sl.y * Q + xt) * Q, we);
#pragma unroll
      for (int q = 0; q < Q; ++q) sr[q] = (k == k0) ? we[q] : sr[q] + we[q];
    }
    return;
  }
  for (uint32_t k = k0; k < k1; k += U) {
    uint2 sl[U];
#pragma unroll
    for (int u = 0; u < U; ++u) sl[u] = a.slots[min(k + (uint32_t)u, k1 - 1u)];
    uint32_t xt[U];
#pragma unroll
    for (int u = 0; u < U; ++u) xt[u] = a.state[(size_t)sl[u].x * a.Cp + c];
    float we[U][Q];
#pragma unroll
    for (int u = 0; u < U; ++u) load_row<Q>(w + ((size_t)sl[u].y * Q + xt[u]) * Q, we[u]);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (k + u < k1) {
#pragma unroll
        for (int q = 0; q < Q; ++q) sr[q] = (k + u == k0) ? we[u][q] : sr[q] + we[u][q];
      }
    }
  }
}

// Generic kernel: any slot counts; a u-role slot reads its column of W as a
// row of the transposed copy.
// Sites per whole-keystream-block run, and the split of such a run into G
// parts of 4 sites for the generic kernel: a run of lcm(Q, 16) / Q sites
// starts on a ChaCha8 block, and a part's words start at a fixed offset into
// its first block, known at compile time per part.  With 16 or 8 sites per
// run (odd Q, or Q = 2 mod 4) one lane per run left few waves and long
// serial work; each part is a lane of its own (the block holding a part's
// first and last words may be computed by two lanes).
template <int Q>
struct PottsRuns {
  static constexpr int SG = Q * 16 / gcd_c(Q, 16) / Q;  // sites per run
  static constexpr int G = SG > 4 ? SG / 4 : 1;         // parts per run
  static constexpr int S = SG / G;                      // sites per part
};

// U: slots per group in role_rows, 1 for programs with at most 6 slots per
// free position on average (a 512^2 torus, 4 per site: grouping cost it
// 15-28 %), else 4 for q <= 8 and 2 above (Erdos-Renyi Potts, 262K nodes,
// mean degree 12: q = 5 1051 -> 722 us per sweep, q = 8 708 -> 570 us)
template <int Q, int U>
__global__ __launch_bounds__(256) void potts_half_kernel(PottsArgs a) {
  using R = PottsRuns<Q>;
  constexpr int S = R::S;
  const uint32_t item = blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= a.n_items) return;
  // part g of every run: items [g * items_per_part, (g + 1) * items_per_part),
  // so that g is the same across a wave
  const uint32_t g = R::G > 1 ? item / a.items_per_part : 0u;
  const uint32_t local = item - g * a.items_per_part;
  const uint32_t run = fdiv(local, a.div_c);
  const uint32_t c = local - run * a.C;
  if (run * (uint32_t)R::SG >= a.n_b) return;
  uint32_t key[8];
  load_key8(a.keys, c, key);
  const uint64_t ctr_run = (uint64_t)run * R::SG * Q / 16u;
  uint32_t blk[16];
  int have = -1;
  static_for<R::G>([&](auto g_c) {
    constexpr int GI = decltype(g_c)::value;
    if (g != (uint32_t)GI) return;
    constexpr int W0 = GI * S * Q;  // the part's first word within the run
    const uint64_t ctr0 = ctr_run + W0 / 16;
    const uint32_t i_begin = run * R::SG + GI * S;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const uint32_t i = i_begin + s;
      const bool live = i < a.n_b;
      const uint32_t pos = a.blk_off + (live ? i : 0u);
      float th[Q];
      load_row<Q>(a.bias + (size_t)pos * Q, th);
      if (a.has_edges) {
        const uint32_t s0 = a.row_off[pos], s1 = a.uend[pos], s2 = a.row_off[pos + 1];
        float su[Q], sv[Q];
        // column x_v of W[e]: row x_v of the transposed copy, contiguous
        role_rows<Q, U>(a, c, s0, s1, a.Wt, su);
#pragma unroll
        for (int q = 0; q < Q; ++q) th[q] = th[q] + su[q];
        role_rows<Q, U>(a, c, s1, s2, a.W, sv);  // row x_u of W[e]
#pragma unroll
        for (int q = 0; q < Q; ++q) th[q] = th[q] + sv[q];
      }
      const uint32_t arg = potts_pick<Q, W0 % 16>(th, s, key, ctr0, blk, have);
      if (live) a.out[(size_t)i * a.Cp + c] = (uint8_t)arg;
    }
  });
}

// Theta of categories q0 .. q0 + 15 of free position pos for chain c
// (entries outside 0..Q-1 are ignored by the caller): ((0 + b) + sum_u) +
// sum_v, each role summed over its slots in order, as in the generic kernel.
// s0, s1, s2 delimit the position's u-role and v-role slots; ro holds the row
// offsets (edge * Q + x_t) * Q of its first four slots.  AL (load_chunk16):
// 16 for Q a multiple of 16, 4 for Q a multiple of 4, 2 for even Q, else 1.
template <int AL, class T>
__device__ __forceinline__ void wide_theta(const PottsArgs &a, const T *state, uint32_t Q,
                                           uint32_t pos, uint32_t c, uint32_t s0, uint32_t s1,
                                           uint32_t s2, const uint64_t (&ro)[4], int32_t q0,
                                           float (&th)[16]) {
  load_chunk16<AL>(a.bias + (size_t)pos * Q, q0, Q, th);
  for (int role = 0; role < 2; ++role) {
    const uint32_t k0 = role ? s1 : s0, k1 = role ? s2 : s1;
    if (k0 == k1) continue;  // an empty role adds nothing: theta is never -0 (bias is 0 + b)
    // u-role: column x_v of W[e], row x_v of the transposed copy
    const float *w = role ? a.W : a.Wt;
    float sr[16];
    for (uint32_t k = k0; k < k1; ++k) {
      const uint32_t j = k - s0;
      uint64_t off;
      if (j < 4u) {
        off = j == 0 ? ro[0] : j == 1 ? ro[1] : j == 2 ? ro[2] : ro[3];
      } else {
        const uint2 sl = a.slots[k];
        off = ((uint64_t)sl.y * Q + state[(size_t)sl.x * a.Cp + c]) * Q;
      }
      float we[16];
      load_chunk16<AL>(w + off, q0, Q, we);
#pragma unroll
      for (int t = 0; t < 16; ++t) sr[t] = (k == k0) ? we[t] : sr[t] + we[t];
    }
#pragma unroll
    for (int t = 0; t < 16; ++t) th[t] = th[t] + sr[t];
  }
}

// The slot range of free position pos and the row offsets of its first four
// slots for chain c (read once, used for every keystream block).
template <class T>
__device__ __forceinline__ void wide_slots(const PottsArgs &a, const T *state, uint32_t Q,
                                           uint32_t pos, uint32_t c, uint32_t &s0, uint32_t &s1,
                                           uint32_t &s2, uint64_t (&ro)[4]) {
  s0 = s1 = s2 = 0u;
  if (a.has_edges) {
    s0 = a.row_off[pos];
    s1 = a.uend[pos];
    s2 = a.row_off[pos + 1];
  }
  // (q = 32 on a 256^2 lattice: 133 -> 112 us per launch for reading them once)
#pragma unroll
  for (uint32_t j = 0; j < 4; ++j) {
    ro[j] = 0;
    if (s0 + j < s2) {
      const uint2 sl = a.slots[s0 + j];
      ro[j] = ((uint64_t)sl.y * Q + state[(size_t)sl.x * a.Cp + c]) * Q;
    }
  }
}

// Wide kernel (16 < Q <= 65536): one lane per (site, chain).  The site's Q
// categories go one keystream block at a time (wide_pick), so a lane holds 16
// of them; slot records and tail bytes past a site's fourth slot are read
// again for every block (they stay in the caches).
// T: the state's element, uint8_t (q <= 256) or uint16_t (q up to 65536).
template <int AL, class T = uint8_t>
__global__ __launch_bounds__(256) void potts_wide_kernel(PottsArgs a, uint32_t Q) {
  const T *state = reinterpret_cast<const T *>(a.state);
  const uint32_t item = blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= a.n_items) return;
  const uint32_t i = fdiv(item, a.div_c);
  const uint32_t c = item - i * a.C;
  uint32_t key[8];
  load_key8(a.keys, c, key);
  const uint32_t pos = a.blk_off + i;
  uint32_t s0, s1, s2;
  uint64_t ro[4];
  wide_slots(a, state, Q, pos, c, s0, s1, s2, ro);
  const uint32_t arg = wide_pick(Q, (uint64_t)i * Q, key, [&](uint32_t, int32_t q0, float(&th)[16]) {
    wide_theta<AL>(a, state, Q, pos, c, s0, s1, s2, ro, q0, th);
  });
  reinterpret_cast<T *>(a.out)[(size_t)i * a.Cp + c] = (T)arg;
}

// Wave kernel for few (site, chain) items with many categories each
// (potts_wave_pays; Q > 256): one wave per item, the lanes splitting the
// site's keystream blocks (wave_pick).
template <int AL, class T>
__global__ __launch_bounds__(256) void potts_wave_kernel(PottsArgs a, uint32_t Q) {
  const T *state = reinterpret_cast<const T *>(a.state);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t item = blockIdx.x * 4u + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (item >= a.n_items) return;  // wave-uniform
  const uint32_t i = fdiv(item, a.div_c);
  const uint32_t c = item - i * a.C;
  uint32_t key[8];
  load_key8(a.keys, c, key);
  const uint32_t pos = a.blk_off + i;
  uint32_t s0, s1, s2;
  uint64_t ro[4];
  wide_slots(a, state, Q, pos, c, s0, s1, s2, ro);
  const uint32_t out = wave_pick(Q, (uint64_t)i * Q, key, lane, [&](uint32_t, int32_t q0, float(&th)[16]) {
    wide_theta<AL>(a, state, Q, pos, c, s0, s1, s2, ro, q0, th);
  });
  if (lane == 0u) reinterpret_cast<T *>(a.out)[(size_t)i * a.Cp + c] = (T)out;
}

// Role-padded kernel (Q a multiple of 4, at most M u-role and M v-role slots
// per position): every site reads M + M slot records, their tails' bytes
// and one contiguous weight row each (row x_v of W[e]^T for the u-role, row
// x_u of W[e] for the v-role), all with static indices, so each stage's loads
// issue together.  Padding slots (edge E, whose rows are zero) follow a
// position's real slots of each role and are skipped: adding +0 would change
// no sum.  theta is the reference's ((0 + b) + sum_u) + sum_v with each sum
// started at its first slot (and 0 for a role without slots).
template <int Q, int M, bool LDSW>
__global__ __launch_bounds__(256) void potts_pad_kernel(PottsArgs a) {
  // LDSW (chains a multiple of 32, so each half-wave holds one run): the
  // half-wave stages its site's 2M weight matrices in LDS with coalesced
  // loads (real slots only), and each lane reads its rows from there, so a
  // matrix passes the texture unit once per site instead of once per slot
  // row gather (config 4: 55 us per launch against 60 us)
  __shared__ float4 wst[LDSW ? 8 * 2 * M * Q * Q / 4 : 1];
  float4 *const wh = wst + (LDSW ? (threadIdx.x >> 5) * (2 * M * Q * Q / 4) : 0);
  constexpr int WORDS = Q * 16 / gcd_c(Q, 16);
  constexpr int S = WORDS / Q;
  constexpr int Q4 = Q / 4;
  const uint32_t item = blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= a.n_items) return;
  const uint32_t run = fdiv(item, a.div_c);
  const uint32_t c = item - run * a.C;
  const uint32_t i_begin = run * S;
  constexpr bool PRE = WORDS == 16;  // one keystream block per lane
  // PRE: the expanded stream key (key_expand) for the block, and the raw key
  // reloaded only for an exact re-draw; otherwise the raw key for potts_pick
  uint32_t key[PRE ? KEY_WORDS : 8];
  if constexpr (PRE)
    load_keyx(a.keys, c, key);
  else
    load_key8(a.keys, c, key);
  const uint64_t ctr0 = (uint64_t)i_begin * Q / 16u;
  uint32_t blk[16];
  int have = -1;
  float gs[16];

  static_for<S>([&](auto s_c) {
    constexpr int s = decltype(s_c)::value;
    const uint32_t i = i_begin + s;
    const bool live = i < a.n_b;
    const uint32_t pos = a.blk_off + (live ? i : 0u);
    uint32_t tail[2 * M], edge[2 * M], xt[2 * M];
#pragma unroll
    for (int j = 0; j < M; ++j) {
      const uint4 r = a.pslots[(size_t)pos * M + j];
      tail[2 * j] = r.x;
      edge[2 * j] = r.y;
      tail[2 * j + 1] = r.z;
      edge[2 * j + 1] = r.w;
    }
    if constexpr (PRE && s == 0) {
      // the keystream block and its scores while the slot records are in
      // flight (ctr0 = i_begin * Q / 16 < n_b < 2^32)
      chacha_block_pre<8>(key, (uint32_t)ctr0, blk);
#pragma unroll
      for (int w = 0; w < 16; ++w) gs[w] = gumbel_fast(blk[w]);
#pragma unroll
      for (int w = 0; w < 16; ++w) asm volatile("" : "+v"(gs[w]));
    }
    // theta of the site.  CMP (a wave whose sites all have at most two slots
    // per role, as interior sites of a lattice): slots 2.. of each role are
    // padding for every lane, so their tail bytes, matrix copies and rows are
    // skipped altogether (config 4: 2 % less time per launch)
    float th[Q];
    auto work = [&](auto cmp_c) {
      constexpr bool CMP = decltype(cmp_c)::value;
      if constexpr (LDSW) {
        // 32-bit offsets (potts_narrow): tail * Cp in 24-bit multiplies
#pragma unroll
        for (int j = 0; j < 2 * M; ++j)
          if (!CMP || j % M < 2) xt[j] = a.state[__umul24(tail[j], a.Cp) + c];
      } else {
#pragma unroll
        for (int j = 0; j < 2 * M; ++j) xt[j] = a.state[(size_t)tail[j] * a.Cp + c];
      }
      if constexpr (LDSW) {
        // The half-wave's 32 lanes copy the site's 2M matrices, F float4 each:
        // pass k takes float4 f = l + 32k, of matrix j = f / F.  Padding slots
        // copy the all-zero matrix of edge E (never read back), so every lane
        // loads unconditionally and the loads of all passes are in flight
        // together.
        constexpr int F = Q * Q / 4;  // float4 per matrix
        constexpr int R = 32 / F;     // matrices per pass
        constexpr int NF = 2 * M * F;
        constexpr int NK = (NF + 31) / 32;
        const uint32_t l = threadIdx.x & 31u;
        const char *const wtb = reinterpret_cast<const char *>(a.Wt);
        const char *const wb = reinterpret_cast<const char *>(a.W);
#pragma unroll
        for (int k = 0; k < NK; ++k) {
          // (a pass of padding matrices only)
          if (CMP && R <= M && (k * R) % M >= 2 && (k * R + R - 1) % M >= 2) continue;
          // a chain of selects, each step hidden from the optimiser: it
          // would otherwise turn the chain into a load from a private copy of
          // edge[] indexed by l / F (scratch memory)
          uint32_t e = edge[k * R];
#pragma unroll
          for (int r = 1; r < R; ++r)
            if (k * R + r < 2 * M) {
              e = l / F == (uint32_t)r ? edge[k * R + r] : e;
              asm("" : "+v"(e));
            }
          const uint32_t off = e * (uint32_t)(Q * Q * 4) + (l % F) * 16u;
          const char *base;
          if constexpr (M % R == 0)
            base = k * R < M ? wtb : wb;  // a pass copies matrices of one role
          else
            base = k * R + l / F < (uint32_t)M ? wtb : wb;
          // a lane past the last matrix (NF < 32) loads a real one and stores nothing
          const float4 v = *reinterpret_cast<const float4 *>(base + off);
          if (NF % 32 == 0 || l + 32u * k < (uint32_t)NF) wh[l + 32u * k] = v;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
      float su[Q], sv[Q];
      const float4 *bp = reinterpret_cast<const float4 *>(a.bias + (size_t)pos * Q);
#pragma unroll
      for (int t = 0; t < Q4; ++t) {
        const float4 v = bp[t];
        th[4 * t] = v.x;
        th[4 * t + 1] = v.y;
        th[4 * t + 2] = v.z;
        th[4 * t + 3] = v.w;
      }
#pragma unroll
      for (int q = 0; q < Q; ++q) su[q] = sv[q] = 0.0f;
#pragma unroll
      for (int j = 0; j < 2 * M; ++j) {
        // padding slots (edge E, all zeros) are skipped: adding +0 changes no sum
        if (CMP && j % M >= 2) continue;
        if (edge[j] != a.n_edges) {
          const float4 *rp = LDSW ? wh + (j * Q + xt[j]) * (Q / 4)
                                  : reinterpret_cast<const float4 *>(
                                        (j < M ? a.Wt : a.W) + ((size_t)edge[j] * Q + xt[j]) * Q);
          float row[Q];
#pragma unroll
          for (int t = 0; t < Q4; ++t) {
            const float4 v = rp[t];
            row[4 * t] = v.x;
            row[4 * t + 1] = v.y;
            row[4 * t + 2] = v.z;
            row[4 * t + 3] = v.w;
          }
#pragma unroll
          for (int q = 0; q < Q; ++q) {
            if (j == 0) su[q] = row[q];
            else if (j < M) su[q] = su[q] + row[q];
            else if (j == M) sv[q] = row[q];
            else sv[q] = sv[q] + row[q];
          }
        }
      }
#pragma unroll
      for (int q = 0; q < Q; ++q) th[q] = (th[q] + su[q]) + sv[q];
    };
    bool compact = false;
    if constexpr (M == 4 && LDSW) {
      bool pad = true;
#pragma unroll
      for (int j = 0; j < 2 * M; ++j)
        if (j % M >= 2) pad = pad && edge[j] == a.n_edges;
      compact = __builtin_amdgcn_ballot_w64(!pad) == 0u;  // wave-uniform
    }
    if (compact) work(std::integral_constant<bool, true>{});
    else work(std::integral_constant<bool, false>{});
    uint32_t arg;
    if constexpr (PRE)
      arg = potts_pick_pre<Q>(th, s, gs, a.keys, c, ctr0);
    else
      arg = potts_pick<Q>(th, s, key, ctr0, blk, have);
    if (live) a.out[(size_t)i * a.Cp + c] = (uint8_t)arg;
    if constexpr (LDSW) {
      // this site's rows are read before the next site's matrices land
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  });
}

// State import / export: caller layout [C][n_b] (u8, or f32 category values)
// <-> [n_total][Cp] bytes.  The sweep kernels index the q x q weight rows
// with the stored category, so only 0..q-1 (u8), or the floats 0.0..q-1.0,
// are accepted; any other value is stored as 0 and raises *bad.
template <class T>
__global__ void potts_pack_kernel(const void *__restrict__ src, int dtype, uint32_t C,
                                  uint32_t n_b, uint32_t Cp, uint32_t q, T *__restrict__ dst,
                                  uint32_t *__restrict__ bad) {
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (uint64_t)C * n_b) return;
  const uint32_t i = (uint32_t)(t / C), c = (uint32_t)(t - (uint64_t)i * C);
  const size_t off = (size_t)c * n_b + i;
  uint32_t v;
  bool ok;
  if (dtype == THRML_DTYPE_U8) {
    v = reinterpret_cast<const uint8_t *>(src)[off];
    ok = v < q;
  } else {
    const float x = reinterpret_cast<const float *>(src)[off];
    ok = x >= 0.0f && x < (float)q && x == __builtin_floorf(x);
    v = ok ? (uint32_t)x : 0u;
  }
  if (!ok) {
    v = 0u;
    *bad = 1u;
  }
  dst[(size_t)i * Cp + c] = (T)v;
}

template <class T>
__global__ void potts_unpack_kernel(const T *__restrict__ srcb, int dtype, uint32_t C,
                                    uint32_t n_b, uint32_t Cp, void *__restrict__ dst) {
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (uint64_t)C * n_b) return;
  const uint32_t c = (uint32_t)(t / n_b), i = (uint32_t)(t - (uint64_t)c * n_b);
  const T v = srcb[(size_t)i * Cp + c];
  if (dtype == THRML_DTYPE_U8)
    reinterpret_cast<uint8_t *>(dst)[t] = (uint8_t)v;  // (u8 reads of q > 256 are refused)
  else
    reinterpret_cast<float *>(dst)[t] = (float)v;
}

static inline uint32_t cdiv32(uint64_t a, uint64_t b) { return (uint32_t)((a + b - 1) / b); }

template <int Q>
static void launch_q(const PottsArgs &a, uint32_t pm, uint32_t mean_slots, hipStream_t s) {
  const dim3 grid(cdiv32(a.n_items, 256));
  if constexpr (Q % 4 == 0) {
    // LDS staging: 2M matrices of Q*Q floats per half-wave, 16 KiB per
    // workgroup at Q = 8 (larger Q stays on the global-memory rows)
    constexpr bool LQ = Q <= 8;
    const bool lds = LQ && a.C % 32u == 0u && a.narrow;
    if (pm == 2u) {
      if (lds) hipLaunchKernelGGL((potts_pad_kernel<Q, 2, LQ>), grid, dim3(256), 0, s, a);
      else hipLaunchKernelGGL((potts_pad_kernel<Q, 2, false>), grid, dim3(256), 0, s, a);
      return;
    }
    if (pm == 4u) {
      if (lds) hipLaunchKernelGGL((potts_pad_kernel<Q, 4, LQ>), grid, dim3(256), 0, s, a);
      else hipLaunchKernelGGL((potts_pad_kernel<Q, 4, false>), grid, dim3(256), 0, s, a);
      return;
    }
  }
  // generic kernel: G parts of every run, each part's items padded to whole waves
  using R = PottsRuns<Q>;
  PottsArgs b = a;
  const uint64_t per = ((uint64_t)cdiv32(a.n_b, R::SG) * a.C + 63u) & ~63ull;
  b.items_per_part = (uint32_t)per;
  b.n_items = (uint32_t)(per * R::G);
  const dim3 g(cdiv32(b.n_items, 256));
  if (mean_slots <= 6u) hipLaunchKernelGGL((potts_half_kernel<Q, 1>), g, dim3(256), 0, s, b);
  else hipLaunchKernelGGL((potts_half_kernel<Q, Q <= 8 ? 4 : 2>), g, dim3(256), 0, s, b);
}

int launch_potts_half(thrml_prog *p, thrml_state *st, uint32_t b, const uint32_t *d_keys) {
  const uint32_t n_b = (uint32_t)(p->blk_off[b + 1] - p->blk_off[b]);
  const uint32_t Q = p->q;
  const uint32_t g = gcd_c((int)Q, 16);
  const uint32_t S = 16u / g;  // lcm(Q, 16) / Q
  PottsArgs a;
  a.state = st->cat.as<uint8_t>();
  // a staged block's new categories replace the old ones after its
  // superblock (crates/thrml-samplers/src/sampling.rs:39-60)
  uint64_t soff = 0, swidth = 0;
  a.out = stage_target(p, b, &soff, &swidth)
              ? st->scratch.as<uint8_t>() + (size_t)soff * st->Cp * p->cat_bytes
              : st->cat.as<uint8_t>() + (size_t)p->blk_off[b] * st->Cp * p->cat_bytes;
  a.row_off = p->row_off.as<uint32_t>();
  a.uend = p->uend.as<uint32_t>();
  a.slots = p->slots.as<uint2>();
  a.bias = p->bias_w.as<float>();
  a.W = p->wts.as<float>();
  a.Wt = p->wts_t.as<float>();
  a.pslots = p->pm ? p->pslots.as<uint4>() : nullptr;
  a.keys = d_keys;
  a.n_b = n_b;
  a.blk_off = (uint32_t)p->blk_off[b];
  a.C = st->C;
  a.div_c = make_fastdiv(st->C);
  a.Cp = st->Cp;
  // (site run, chain) items are indexed in 32 bits and divided by C with a
  // reciprocal that is exact below 2^31
  // (the generic kernel's parts of 4 sites, padded to whole waves, stay
  // within the same bound: (n_b / 4 + 64) x C < 2^31 for any block it runs)
  if ((uint64_t)cdiv32(n_b, S) * st->C >= (1ull << 31) ||
      ((uint64_t)cdiv32(n_b, 4) + 64u) * st->C >= (1ull << 31))
    return fail(THRML_EINVAL, "categorical block too large: (sites / runs) x chains must stay below 2^31");
  a.n_items = cdiv32(n_b, S) * st->C;
  a.has_edges = p->n_edges ? 1u : 0u;
  a.n_edges = (uint32_t)p->n_edges;
  a.narrow = potts_narrow(p->n_total, st->Cp, p->n_edges, Q) ? 1u : 0u;
  hipEvent_t t0 = nullptr;
  if (p->ctx->time_begin(0, &t0)) return THRML_EHIP;
  hipStream_t s = p->ctx->stream;
  switch (Q) {
    case 2: launch_q<2>(a, p->pm, p->mean_slots, s); break;
    case 3: launch_q<3>(a, p->pm, p->mean_slots, s); break;
    case 4: launch_q<4>(a, p->pm, p->mean_slots, s); break;
    case 5: launch_q<5>(a, p->pm, p->mean_slots, s); break;
    case 6: launch_q<6>(a, p->pm, p->mean_slots, s); break;
    case 7: launch_q<7>(a, p->pm, p->mean_slots, s); break;
    case 8: launch_q<8>(a, p->pm, p->mean_slots, s); break;
    case 9: launch_q<9>(a, p->pm, p->mean_slots, s); break;
    case 10: launch_q<10>(a, p->pm, p->mean_slots, s); break;
    case 11: launch_q<11>(a, p->pm, p->mean_slots, s); break;
    case 12: launch_q<12>(a, p->pm, p->mean_slots, s); break;
    case 13: launch_q<13>(a, p->pm, p->mean_slots, s); break;
    case 14: launch_q<14>(a, p->pm, p->mean_slots, s); break;
    case 15: launch_q<15>(a, p->pm, p->mean_slots, s); break;
    case 16: launch_q<16>(a, p->pm, p->mean_slots, s); break;
    default: {
      if (Q > (p->cat_bytes == 2 ? POTTS_WIDE_MAX_Q : POTTS_MAX_Q))
        return fail(THRML_EINVAL, "q must lie in 2..65536");
      // one lane per (site, chain)
      if ((uint64_t)n_b * st->C >= (1ull << 31))
        return fail(THRML_EINVAL, "categorical block too large: sites x chains must stay below 2^31");
      a.n_items = n_b * st->C;
      const dim3 grid(cdiv32(a.n_items, 256));
      if (potts_wave_pays(Q, a.n_items)) {
        // few items for their categories (two-byte states): one wave per item
        static_assert(POTTS_WAVE_MIN_Q > POTTS_MAX_Q, "the wave kernel reads two-byte states");
        const dim3 wg(cdiv32(a.n_items, 4));
        if (Q % 16 == 0) hipLaunchKernelGGL((potts_wave_kernel<16, uint16_t>), wg, dim3(256), 0, s, a, Q);
        else if (Q % 4 == 0) hipLaunchKernelGGL((potts_wave_kernel<4, uint16_t>), wg, dim3(256), 0, s, a, Q);
        else if (Q % 2 == 0) hipLaunchKernelGGL((potts_wave_kernel<2, uint16_t>), wg, dim3(256), 0, s, a, Q);
        else hipLaunchKernelGGL((potts_wave_kernel<1, uint16_t>), wg, dim3(256), 0, s, a, Q);
      } else if (p->cat_bytes == 2) {
        if (Q % 16 == 0) hipLaunchKernelGGL((potts_wide_kernel<16, uint16_t>), grid, dim3(256), 0, s, a, Q);
        else if (Q % 4 == 0) hipLaunchKernelGGL((potts_wide_kernel<4, uint16_t>), grid, dim3(256), 0, s, a, Q);
        else if (Q % 2 == 0) hipLaunchKernelGGL((potts_wide_kernel<2, uint16_t>), grid, dim3(256), 0, s, a, Q);
        else hipLaunchKernelGGL((potts_wide_kernel<1, uint16_t>), grid, dim3(256), 0, s, a, Q);
      } else if (Q % 16 == 0) hipLaunchKernelGGL(potts_wide_kernel<16>, grid, dim3(256), 0, s, a, Q);
      else if (Q % 4 == 0) hipLaunchKernelGGL(potts_wide_kernel<4>, grid, dim3(256), 0, s, a, Q);
      else if (Q % 2 == 0) hipLaunchKernelGGL(potts_wide_kernel<2>, grid, dim3(256), 0, s, a, Q);
      else hipLaunchKernelGGL(potts_wide_kernel<1>, grid, dim3(256), 0, s, a, Q);
    }
  }
  THRML_HIP(hipGetLastError());
  return p->ctx->time_end(0, t0);
}

// Program creation: the transposed copy of the edge weights, wt[e][c][x] =
// w[e][x][c] (a u-role slot reads row x_v of it), and the all-zero padding
// edge E of both arrays when the program has one (n_w > n_edges * q * q).
__global__ void potts_weights_kernel(float *__restrict__ w, float *__restrict__ wt, uint64_t n_edges,
                                     uint32_t q, uint64_t n_w) {
  const uint64_t qq = (uint64_t)q * q;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; t < n_w; t += stride) {
    const uint64_t e = t / qq;
    if (e >= n_edges) {
      w[t] = 0.0f;
      wt[t] = 0.0f;
      continue;
    }
    const uint64_t r = t - e * qq;
    const uint64_t c = r / q, x = r - c * q;
    wt[t] = w[e * qq + x * q + c];
  }
}

int launch_potts_weights(thrml_ctx *ctx, float *w, float *wt, uint64_t n_edges, uint32_t q,
                         uint64_t n_w) {
  if (n_w == 0) return THRML_OK;
  const uint64_t blocks = std::min<uint64_t>((n_w + 255) / 256, 1u << 20);
  hipLaunchKernelGGL(potts_weights_kernel, dim3((uint32_t)blocks), dim3(256), 0, ctx->stream, w, wt,
                     n_edges, q, n_w);
  THRML_HIP(hipGetLastError());
  return THRML_OK;
}

int launch_potts_pack(thrml_state *st, uint32_t b, const void *d_src, int dtype, uint32_t *d_bad) {
  thrml_prog *p = st->prog;
  const uint32_t n_b = (uint32_t)(p->blk_off[b + 1] - p->blk_off[b]);
  const uint64_t n = (uint64_t)st->C * n_b;
  if (n == 0) return THRML_OK;
  const size_t at = (size_t)p->blk_off[b] * st->Cp;
  if (p->cat_bytes == 2)
    hipLaunchKernelGGL(potts_pack_kernel<uint16_t>, dim3(cdiv32(n, 256)), dim3(256), 0, p->ctx->stream,
                       d_src, dtype, st->C, n_b, st->Cp, block_q(p, b), st->cat.as<uint16_t>() + at, d_bad);
  else
    hipLaunchKernelGGL(potts_pack_kernel<uint8_t>, dim3(cdiv32(n, 256)), dim3(256), 0, p->ctx->stream,
                       d_src, dtype, st->C, n_b, st->Cp, block_q(p, b), st->cat.as<uint8_t>() + at, d_bad);
  THRML_HIP(hipGetLastError());
  return THRML_OK;
}

int launch_potts_unpack(thrml_state *st, uint32_t b, void *d_dst, int dtype) {
  thrml_prog *p = st->prog;
  const uint32_t n_b = (uint32_t)(p->blk_off[b + 1] - p->blk_off[b]);
  const uint64_t n = (uint64_t)st->C * n_b;
  if (n == 0) return THRML_OK;
  const size_t at = (size_t)p->blk_off[b] * st->Cp;
  if (p->cat_bytes == 2)
    hipLaunchKernelGGL(potts_unpack_kernel<uint16_t>, dim3(cdiv32(n, 256)), dim3(256), 0,
                       p->ctx->stream, st->cat.as<uint16_t>() + at, dtype, st->C, n_b, st->Cp, d_dst);
  else
    hipLaunchKernelGGL(potts_unpack_kernel<uint8_t>, dim3(cdiv32(n, 256)), dim3(256), 0,
                       p->ctx->stream, st->cat.as<uint8_t>() + at, dtype, st->C, n_b, st->Cp, d_dst);
  THRML_HIP(hipGetLastError());
  return THRML_OK;
}

}  // namespace thrml
