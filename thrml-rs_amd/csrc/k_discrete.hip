// k_discrete.hip -- block Gibbs half-sweep and energies of programs over
// general discrete factors (gfx950).
//
// One launch updates one free block of every chain.  Spin blocks follow
// SpinGibbsConditional (crates/thrml-samplers/src/spin_gibbs.rs:512-595):
//   gamma = (((0 + S_1) + S_2) + ...), S_g the sum of group g's slots in
//   order, a slot contributing +-w (w = row entry at the first categorical
//   tail's category, or entry 0; the sign the product of 2 s - 1 over the
//   spin tails); s' = (u <= sigmoid(2 gamma)), u from keystream word i.
// Categorical blocks follow CategoricalGibbsConditional
// (crates/thrml-samplers/src/softmax.rs:586-710):
//   theta[c] accumulated alike with +-W'[c] or +-W'[c][x];
//   x' = first argmax_c(theta[c] + Gumbel), keystream word i * q + c.
// State: one byte per (position, chain), chains fastest ([n_total][Cp]).
// Work split: a lane takes one chain and a run of S sites: 4 for spins (a
// quarter of a keystream block), lcm(q, 16) / q for categories (whole
// blocks); consecutive lanes are consecutive chains, so a site's slot
// records are read by all of its chains at once.  Spin sites are summed four
// at a time with their slots interleaved.  q = 17..256: one categorical site
// per lane, its categories one keystream block at a time
// (discrete_wide_kernel).  The generic path: the
// benchmarked Ising and categorical programs have their own kernels.
#include "dev_util.hpp"
#include "internal.hpp"

namespace thrml {

struct DiscArgs {
  const uint8_t *state;     // [n_total][Cp]
  uint8_t *out;             // new values of this block: [n_b][Cp] (in place or staged)
  const uint32_t *row_off;  // [nf + 1]
  const uint4 *slots;       // {weight offset, categorical tail | DISC_NONE, first spin tail, flags}
  const uint32_t *sp;       // spin tail positions
  const float *W;           // all factors' weights, flat
  const uint32_t *keys;     // [G*64][KEY_WORDS] stream keys of this (sweep, block)
  uint32_t n_b, blk_off, C, Cp, n_items;
  uint32_t items_per_part;  // items of one part of every run (a multiple of 64 with parts)
  FastDiv div_c;            // by C
};

constexpr int disc_gcd(int a, int b) { return b == 0 ? a : disc_gcd(b, a % b); }

// S categorical sites of one chain from i_begin on, whose keystream words
// start at word W0 of block ctr0 (W0 < 16)
template <int Q, int S, int W0>
__device__ __forceinline__ void categorical_sites(const DiscArgs &a, uint32_t i_begin, uint32_t c,
                                                  const uint32_t (&key)[8], uint64_t ctr0,
                                                  uint32_t (&blk)[16], int &have) {
  // sites G at a time with their slots interleaved, as in the spin path;
  // for q > 4 the second site's rows and sums cost more registers than the
  // overlap gains (q = 8 on a 512^2 lattice: 106 against 88 us per launch;
  // q = 4: 56 against 73 us)
  constexpr int G = S >= 2 && Q <= 4 ? 2 : 1;
  if constexpr (G == 1) {
    // one site at a time, its slots two at a time: records, then tail bytes,
    // then rows loaded together, the rows added in slot order (a slot past
    // the site's last reloads that slot and adds nothing).  Erdos-Renyi Potts
    // (262K nodes, mean degree 12, 32 chains): q = 5 1228 -> 950 us per
    // sweep, q = 8 810 -> 667 us; four at a time cost config 4's lattice
    // (5 slots per site) 22 %, two at a time gain it 4 %.
    constexpr int U = 2;
    for (int g = 0; g < S; ++g) {
      const uint32_t i = i_begin + (uint32_t)g;
      const uint32_t pos = a.blk_off + min(i, a.n_b - 1u);
      const uint32_t k0 = a.row_off[pos];
      const uint32_t deg = i < a.n_b ? a.row_off[pos + 1] - k0 : 0u;
      float tot[Q], acc[Q];
#pragma unroll
      for (int q = 0; q < Q; ++q) tot[q] = acc[q] = 0.0f;
      for (uint32_t j = 0; j < deg; j += U) {
        uint4 r[U];
#pragma unroll
        for (int v = 0; v < U; ++v) r[v] = a.slots[k0 + min(j + (uint32_t)v, deg - 1u)];
        uint32_t neg[U];
        float wv[U][Q];
#pragma unroll
        for (int v = 0; v < U; ++v) {
          const uint32_t nsp = r[v].w & 255u;
          uint32_t ng = 0u;
          if (nsp >= 1u) ng ^= a.state[(size_t)a.sp[r[v].z] * a.Cp + c] == 0u ? 1u : 0u;
          for (uint32_t t = 1u; t < nsp; ++t)
            ng ^= a.state[(size_t)a.sp[r[v].z + t] * a.Cp + c] == 0u ? 1u : 0u;
          neg[v] = ng;
          const uint32_t x = r[v].y != DISC_NONE ? a.state[(size_t)r[v].y * a.Cp + c] : 0u;
          load_row<Q>(a.W + r[v].x + (((r[v].w >> 9) & 3u) == 2u ? x * Q : 0u), wv[v]);
        }
#pragma unroll
        for (int v = 0; v < U; ++v) {
          if (j + v < deg) {
            const bool first = (r[v].w >> 8) & 1u;
            if (first && j + v != 0u) {
#pragma unroll
              for (int q = 0; q < Q; ++q) tot[q] = tot[q] + acc[q];
            }
#pragma unroll
            for (int q = 0; q < Q; ++q) {
              const float w = neg[v] ? -wv[v][q] : wv[v][q];
              acc[q] = first ? w : acc[q] + w;
            }
          }
        }
      }
      if (deg) {
#pragma unroll
        for (int q = 0; q < Q; ++q) tot[q] = tot[q] + acc[q];
      }
      const uint32_t val = potts_pick<Q, W0 % 16>(tot, g, key, ctr0, blk, have);
      if (i < a.n_b) a.out[(size_t)i * a.Cp + c] = (uint8_t)val;
    }
    return;
  }
  for (int g = 0; g < S; g += G) {
    uint32_t k0[G], deg[G], mx = 0u;
    float tot[G][Q], acc[G][Q];
#pragma unroll
    for (int u = 0; u < G; ++u) {
      const uint32_t i = i_begin + (uint32_t)(g + u);
      const uint32_t pos = a.blk_off + min(i, a.n_b - 1u);
      k0[u] = a.row_off[pos];
      deg[u] = i < a.n_b ? a.row_off[pos + 1] - k0[u] : 0u;
      mx = max(mx, deg[u]);
#pragma unroll
      for (int q = 0; q < Q; ++q) tot[u][q] = acc[u][q] = 0.0f;
    }
    for (uint32_t j = 0; j < mx; ++j) {
      uint4 r[G];
#pragma unroll
      for (int u = 0; u < G; ++u) r[u] = a.slots[k0[u] + min(j, deg[u] ? deg[u] - 1u : 0u)];
      uint32_t neg[G];
      float wv[G][Q];
#pragma unroll
      for (int u = 0; u < G; ++u) {
        const uint32_t nsp = r[u].w & 255u;
        uint32_t ng = 0u;
        if (nsp >= 1u) ng ^= a.state[(size_t)a.sp[r[u].z] * a.Cp + c] == 0u ? 1u : 0u;
        if (nsp >= 2u) ng ^= a.state[(size_t)a.sp[r[u].z + 1u] * a.Cp + c] == 0u ? 1u : 0u;
        for (uint32_t t = 2u; t < nsp; ++t)
          ng ^= a.state[(size_t)a.sp[r[u].z + t] * a.Cp + c] == 0u ? 1u : 0u;
        neg[u] = ng;
        const uint32_t x = r[u].y != DISC_NONE ? a.state[(size_t)r[u].y * a.Cp + c] : 0u;
        // the slot's row of q contiguous floats at entry 0 (axis 0) or x * q
        // (axis 2), 16-byte aligned
        const float *row = a.W + r[u].x + (((r[u].w >> 9) & 3u) == 2u ? x * Q : 0u);
        if constexpr (Q % 4 == 0) {
#pragma unroll
          for (int t = 0; t < Q / 4; ++t) {
            const float4 f = reinterpret_cast<const float4 *>(row)[t];
            wv[u][4 * t] = f.x;
            wv[u][4 * t + 1] = f.y;
            wv[u][4 * t + 2] = f.z;
            wv[u][4 * t + 3] = f.w;
          }
        } else {
#pragma unroll
          for (int q = 0; q < Q; ++q) wv[u][q] = row[q];
        }
      }
#pragma unroll
      for (int u = 0; u < G; ++u) {
        if (j < deg[u]) {
          const bool first = (r[u].w >> 8) & 1u;
          if (first && j != 0u) {
#pragma unroll
            for (int q = 0; q < Q; ++q) tot[u][q] = tot[u][q] + acc[u][q];
          }
#pragma unroll
          for (int q = 0; q < Q; ++q) {
            // w * (+-1) is exactly +-w
            const float v = neg[u] ? -wv[u][q] : wv[u][q];
            acc[u][q] = first ? v : acc[u][q] + v;
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < G; ++u) {
      const uint32_t i = i_begin + (uint32_t)(g + u);
      if (deg[u]) {
#pragma unroll
        for (int q = 0; q < Q; ++q) tot[u][q] = tot[u][q] + acc[u][q];
      }
      const uint32_t val = potts_pick<Q, W0 % 16>(tot[u], g + u, key, ctr0, blk, have);
      if (i < a.n_b) a.out[(size_t)i * a.Cp + c] = (uint8_t)val;
    }
  }
}

// q = 4 is held to 64 VGPRs, 8 waves per SIMD: it fits them without spilling,
// and the compiler's own choice, 67, costs a wave and 7 % per launch
// T: the state's element, uint8_t, or uint16_t in spin blocks of a program
// whose categorical nodes have more than 256 categories (those blocks run the
// wide kernel)
template <int Q, class T = uint8_t>  // Q: 0 spin block, else the categories of a categorical block
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(Q == 4 ? 8 : 1)))
void discrete_half_kernel(DiscArgs a) {
  static_assert(Q == 0 || sizeof(T) == 1, "categorical blocks of Q <= 16 hold one byte per node");
  const T *state = reinterpret_cast<const T *>(a.state);
  // sites per run: spin blocks 4, a quarter of a keystream block (more waves:
  // the sums are latency-bound, and 4-site runs measured 25 % faster than
  // 16-site ones on a 512^2 lattice); categorical blocks lcm(Q, 16) / Q,
  // whole blocks, split into NP parts of 4 sites when that is 8 or 16 (each
  // part a lane, its keystream offset fixed at compile time, one part per
  // wave: items [p * items_per_part, (p + 1) * items_per_part) are part p)
  constexpr int SG = Q == 0 ? 4 : 16 / disc_gcd(Q, 16);
  constexpr int NP = Q != 0 && SG > 4 ? SG / 4 : 1;
  constexpr int S = SG / NP;
  const uint32_t item = blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= a.n_items) return;
  const uint32_t part = NP > 1 ? item / a.items_per_part : 0u;
  const uint32_t local = item - part * a.items_per_part;
  const uint32_t run = fdiv(local, a.div_c);
  const uint32_t c = local - run * a.C;
  if constexpr (NP > 1)
    if (run * (uint32_t)SG >= a.n_b) return;  // padding of a part's items
  uint32_t key[8];
  load_key8(a.keys, c, key);
  uint32_t blk[16];
  int have = -1;
  if constexpr (Q == 0) {
    const uint32_t i_begin = run * S;
    const uint64_t ctr0 = i_begin / 16u;
    chacha_block<8>(key, ctr0, blk);  // the block holding the run's 4 words
    // spin sites four at a time: slot j of the four sites is read together,
    // so that four chains of dependent loads (record, tail position, tail
    // byte, weight) are in flight; each site still sums its slots in order
    static_assert(S == 4, "a spin run is one quarter of a keystream block");
#pragma unroll
    for (int g = 0; g < S; g += 4) {
      uint32_t k0[4], deg[4], mx = 0u;
      float tot[4], acc[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t i = i_begin + (uint32_t)(g + u);
        const uint32_t pos = a.blk_off + min(i, a.n_b - 1u);
        k0[u] = a.row_off[pos];
        deg[u] = i < a.n_b ? a.row_off[pos + 1] - k0[u] : 0u;
        mx = max(mx, deg[u]);
        tot[u] = acc[u] = 0.0f;
      }
      for (uint32_t j = 0; j < mx; ++j) {
        uint4 r[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) r[u] = a.slots[k0[u] + min(j, deg[u] ? deg[u] - 1u : 0u)];
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const uint32_t nsp = r[u].w & 255u;
          uint32_t neg = 0u;
          if (nsp >= 1u) neg ^= state[(size_t)a.sp[r[u].z] * a.Cp + c] == 0u ? 1u : 0u;
          if (nsp >= 2u) neg ^= state[(size_t)a.sp[r[u].z + 1u] * a.Cp + c] == 0u ? 1u : 0u;
          for (uint32_t t = 2u; t < nsp; ++t)
            neg ^= state[(size_t)a.sp[r[u].z + t] * a.Cp + c] == 0u ? 1u : 0u;
          const uint32_t x = r[u].y != DISC_NONE ? state[(size_t)r[u].y * a.Cp + c] : 0u;
          const float w = a.W[r[u].x + x];
          v[u] = neg ? -w : w;  // w * (+-1) is exactly +-w
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          if (j < deg[u]) {
            const bool first = (r[u].w >> 8) & 1u;
            if (first && j != 0u) tot[u] = tot[u] + acc[u];
            acc[u] = first ? v[u] : acc[u] + v[u];
          }
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const uint32_t i = i_begin + (uint32_t)(g + u);
        if (deg[u]) tot[u] = tot[u] + acc[u];
        if (i < a.n_b)
          reinterpret_cast<T *>(a.out)[(size_t)i * a.Cp + c] = spin_decision(tot[u], blk[i & 15u]) ? 1u : 0u;
      }
    }
  } else {
    const uint64_t ctr_run = (uint64_t)run * SG * Q / 16u;
    if constexpr (NP == 1) {
      categorical_sites<Q, S, 0>(a, run * SG, c, key, ctr_run, blk, have);
    } else {
      // (a function, not the lambda's body: a lambda here costs the NP = 1
      // kernels 3 VGPRs, and q = 4 an occupancy step)
      static_for<NP>([&](auto p_c) {
        constexpr int PI = decltype(p_c)::value;
        constexpr int W0 = PI * S * Q;  // the part's first word within the run
        if (part == (uint32_t)PI)
          categorical_sites<Q, S, W0>(a, run * SG + PI * S, c, key, ctr_run + W0 / 16, blk, have);
      });
    }
  }
}

// Categorical blocks with 16 < Q <= 256 categories: one lane per (site,
// chain).  The site's categories go one keystream block at a time
// (wide_pick); for each, the slots are walked again and summed per category
// as above (groups from their first slot, added to theta in order), the
// first four slots' rows and signs kept from one read.  AL (load_chunk16):
// 16 for Q a multiple of 16, 4 for Q a multiple of 4, 2 for even Q (weight
// rows start at multiples of 4 floats), else 1.
// WAVE: one wave per item, its lanes splitting the site's keystream blocks
// (wave_pick; two-byte programs with few items for their categories,
// potts_wave_pays), else one lane per item.
template <int AL, class T = uint8_t, bool WAVE = false>
__global__ __launch_bounds__(256) void discrete_wide_kernel(DiscArgs a, uint32_t Q) {
  const T *state = reinterpret_cast<const T *>(a.state);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t item = WAVE ? blockIdx.x * 4u + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6)
                             : blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= a.n_items) return;
  const uint32_t i = fdiv(item, a.div_c);
  const uint32_t c = item - i * a.C;
  uint32_t key[8];
  load_key8(a.keys, c, key);
  const uint32_t pos = a.blk_off + i;
  const uint32_t k0 = a.row_off[pos], deg = a.row_off[pos + 1] - k0;
  // slot j: its row's offset in W, and its sign (bit 0) and group-start
  // (bit 1) flags
  auto slot = [&](uint32_t j, uint32_t &off, uint32_t &fl) {
    const uint4 r = a.slots[k0 + j];
    const uint32_t nsp = r.w & 255u;
    uint32_t neg = 0u;
    for (uint32_t t = 0; t < nsp; ++t)
      neg ^= state[(size_t)a.sp[r.z + t] * a.Cp + c] == 0u ? 1u : 0u;
    const uint32_t x = r.y != DISC_NONE ? state[(size_t)r.y * a.Cp + c] : 0u;
    off = r.x + (((r.w >> 9) & 3u) == 2u ? x * Q : 0u);
    fl = neg | (((r.w >> 8) & 1u) << 1);
  };
  // the first 4 slots are read once for all blocks
  uint32_t ro[4], rf[4];
#pragma unroll
  for (uint32_t j = 0; j < 4; ++j) {
    ro[j] = rf[j] = 0u;
    if (j < deg) slot(j, ro[j], rf[j]);
  }
  auto theta_chunk = [&](uint32_t, int32_t q0, float (&th)[16]) {
    float acc[16];
#pragma unroll
    for (int t = 0; t < 16; ++t) th[t] = acc[t] = 0.0f;
    for (uint32_t j = 0; j < deg; ++j) {
      uint32_t off, fl;
      if (j < 4u) {
        off = j == 0 ? ro[0] : j == 1 ? ro[1] : j == 2 ? ro[2] : ro[3];
        fl = j == 0 ? rf[0] : j == 1 ? rf[1] : j == 2 ? rf[2] : rf[3];
      } else {
        slot(j, off, fl);
      }
      const bool neg = fl & 1u;
      float wv[16];
      load_chunk16<AL>(a.W + off, q0, Q, wv);
      const bool first = fl & 2u;
      if (first && j != 0u) {
#pragma unroll
        for (int t = 0; t < 16; ++t) th[t] = th[t] + acc[t];
      }
#pragma unroll
      for (int t = 0; t < 16; ++t) {
        const float v = neg ? -wv[t] : wv[t];
        acc[t] = first ? v : acc[t] + v;
      }
    }
    if (deg) {
#pragma unroll
      for (int t = 0; t < 16; ++t) th[t] = th[t] + acc[t];
    }
  };
  if constexpr (WAVE) {
    const uint32_t arg = wave_pick(Q, (uint64_t)i * Q, key, lane, theta_chunk);
    if (lane == 0u) reinterpret_cast<T *>(a.out)[(size_t)i * a.Cp + c] = (T)arg;
  } else {
    const uint32_t arg = wide_pick(Q, (uint64_t)i * Q, key, theta_chunk);
    reinterpret_cast<T *>(a.out)[(size_t)i * a.Cp + c] = (T)arg;
  }
}

static inline uint32_t cdiv32(uint64_t x, uint64_t y) { return (uint32_t)((x + y - 1) / y); }

template <int Q, class T = uint8_t>
static void launch_dq(const DiscArgs &a, hipStream_t s) {
  hipLaunchKernelGGL((discrete_half_kernel<Q, T>), dim3(cdiv32(a.n_items, 256)), dim3(256), 0, s, a);
}

int launch_discrete_half(thrml_prog *p, thrml_state *st, uint32_t b, const uint32_t *d_keys) {
  const uint32_t n_b = (uint32_t)(p->blk_off[b + 1] - p->blk_off[b]);
  const bool spin = !p->blk_kind[b];
  const uint32_t Q = spin ? 0u : p->q;
  const bool wide = Q > 16u;  // one site per lane
  // sites per run and parts per run, as in the kernel
  const uint32_t SG = wide ? 1u : spin ? 4u : 16u / (uint32_t)disc_gcd((int)Q, 16);
  const uint32_t NP = !spin && SG > 4u ? SG / 4u : 1u;
  DiscArgs a;
  a.state = st->cat.as<uint8_t>();
  // a staged block's new values replace the old ones after its superblock
  // (crates/thrml-samplers/src/sampling.rs:39-60)
  uint64_t soff = 0, swidth = 0;
  a.out = stage_target(p, b, &soff, &swidth)
              ? st->scratch.as<uint8_t>() + (size_t)soff * st->Cp * p->cat_bytes
              : st->cat.as<uint8_t>() + (size_t)p->blk_off[b] * st->Cp * p->cat_bytes;
  a.row_off = p->row_off.as<uint32_t>();
  a.slots = p->d_slots.as<uint4>();
  a.sp = p->d_sp.as<uint32_t>();
  a.W = p->d_w.as<float>();
  a.keys = d_keys;
  a.n_b = n_b;
  a.blk_off = (uint32_t)p->blk_off[b];
  a.C = st->C;
  a.div_c = make_fastdiv(st->C);
  a.Cp = st->Cp;
  // (run, chain) items are indexed in 32 bits and divided by C with a
  // reciprocal that is exact below 2^31
  // (parts start on a wave boundary, so that a wave holds one part)
  const uint64_t runs = (uint64_t)cdiv32(n_b, SG) * st->C;
  const uint64_t per = NP > 1 ? (runs + 63u) & ~63ull : runs;
  if (per * NP >= (1ull << 31))
    return fail(THRML_EINVAL, "block too large: (sites / runs) x chains must stay below 2^31");
  a.items_per_part = (uint32_t)per;
  a.n_items = (uint32_t)(per * NP);
  hipEvent_t t0 = nullptr;
  if (p->ctx->time_begin(0, &t0)) return THRML_EHIP;
  hipStream_t s = p->ctx->stream;
  switch (Q) {
    case 0:
      if (p->cat_bytes == 2) launch_dq<0, uint16_t>(a, s);
      else launch_dq<0>(a, s);
      break;
    case 2: launch_dq<2>(a, s); break;
    case 3: launch_dq<3>(a, s); break;
    case 4: launch_dq<4>(a, s); break;
    case 5: launch_dq<5>(a, s); break;
    case 6: launch_dq<6>(a, s); break;
    case 7: launch_dq<7>(a, s); break;
    case 8: launch_dq<8>(a, s); break;
    case 9: launch_dq<9>(a, s); break;
    case 10: launch_dq<10>(a, s); break;
    case 11: launch_dq<11>(a, s); break;
    case 12: launch_dq<12>(a, s); break;
    case 13: launch_dq<13>(a, s); break;
    case 14: launch_dq<14>(a, s); break;
    case 15: launch_dq<15>(a, s); break;
    case 16: launch_dq<16>(a, s); break;
    default: {
      if (Q > (p->cat_bytes == 2 ? POTTS_WIDE_MAX_Q : POTTS_MAX_Q))
        return fail(THRML_EINVAL, "q must lie in 2..65536");
      const dim3 grid(cdiv32(a.n_items, 256));
      if (potts_wave_pays(Q, a.n_items)) {
        // few items for their categories (two-byte states): one wave per item
        const dim3 wg(cdiv32(a.n_items, 4));
        if (Q % 16 == 0) hipLaunchKernelGGL((discrete_wide_kernel<16, uint16_t, true>), wg, dim3(256), 0, s, a, Q);
        else if (Q % 4 == 0) hipLaunchKernelGGL((discrete_wide_kernel<4, uint16_t, true>), wg, dim3(256), 0, s, a, Q);
        else if (Q % 2 == 0) hipLaunchKernelGGL((discrete_wide_kernel<2, uint16_t, true>), wg, dim3(256), 0, s, a, Q);
        else hipLaunchKernelGGL((discrete_wide_kernel<1, uint16_t, true>), wg, dim3(256), 0, s, a, Q);
      } else if (p->cat_bytes == 2) {
        if (Q % 16 == 0) hipLaunchKernelGGL((discrete_wide_kernel<16, uint16_t>), grid, dim3(256), 0, s, a, Q);
        else if (Q % 4 == 0) hipLaunchKernelGGL((discrete_wide_kernel<4, uint16_t>), grid, dim3(256), 0, s, a, Q);
        else if (Q % 2 == 0) hipLaunchKernelGGL((discrete_wide_kernel<2, uint16_t>), grid, dim3(256), 0, s, a, Q);
        else hipLaunchKernelGGL((discrete_wide_kernel<1, uint16_t>), grid, dim3(256), 0, s, a, Q);
      } else if (Q % 16 == 0) hipLaunchKernelGGL(discrete_wide_kernel<16>, grid, dim3(256), 0, s, a, Q);
      else if (Q % 4 == 0) hipLaunchKernelGGL(discrete_wide_kernel<4>, grid, dim3(256), 0, s, a, Q);
      else if (Q % 2 == 0) hipLaunchKernelGGL(discrete_wide_kernel<2>, grid, dim3(256), 0, s, a, Q);
      else hipLaunchKernelGGL(discrete_wide_kernel<1>, grid, dim3(256), 0, s, a, Q);
    }
  }
  THRML_HIP(hipGetLastError());
  return p->ctx->time_end(0, t0);
}

// ---------------------------------------------------------------------------
// Energies: DiscreteEBMFactor::factor_energy (crates/thrml-models/src/discrete_ebm.rs:
// 551-593) summed over the factors, E[c] = -sum_t W[t][x_0][x_1] prod(2 s - 1)
// over the energy terms t (factor rows with every node in a block).  A wave
// takes a chunk of terms for 64 chains (lane = chain) and writes one f64
// partial per chain; reduce_energy adds a chain's partials in a fixed order.
constexpr uint32_t DISC_EN_CHUNK = 256;

struct DiscEnergyArgs {
  const uint8_t *cat;     // [n_total][Cp], one byte per node
  const uint16_t *cat16;  // or two (more than 256 categories): the other is null
  const uint4 *terms;     // two per term
  const uint32_t *tsp;
  const float *W;
  uint64_t n_terms;
  uint32_t n_ch, C, Cp, CG;
  double *part;           // [n_ch][CG * 64]
};

__global__ __launch_bounds__(256) void discrete_energy_kernel(DiscEnergyArgs a) {
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t task = blockIdx.x * 4u + wave;
  if (task >= a.n_ch * a.CG) return;
  const uint32_t g = task / a.n_ch, k = task - g * a.n_ch;
  const uint32_t c = g * 64u + lane;
  const bool live = c < a.C;
  const uint32_t cc = live ? c : 0u;  // dead lanes read chain 0 and add nothing
  auto cat = [&](size_t at) -> uint32_t { return a.cat16 ? a.cat16[at] : a.cat[at]; };
  const uint64_t t0 = (uint64_t)k * DISC_EN_CHUNK;
  const uint64_t t1 = t0 + DISC_EN_CHUNK < a.n_terms ? t0 + DISC_EN_CHUNK : a.n_terms;
  double acc = 0.0;
  for (uint64_t t = t0; t < t1; ++t) {
    const uint4 r0 = a.terms[2 * t], r1 = a.terms[2 * t + 1];
    uint32_t neg = 0u;
    for (uint32_t j = 0; j < r0.z; ++j) neg ^= cat((size_t)a.tsp[r0.y + j] * a.Cp + cc) == 0u ? 1u : 0u;
    uint32_t idx = 0u;
    if (r0.w != DISC_NONE) {
      const uint32_t x0 = cat((size_t)r0.w * a.Cp + cc);
      idx = r1.x != DISC_NONE ? x0 * r1.y + cat((size_t)r1.x * a.Cp + cc) : x0;
    }
    const double v = (double)a.W[r0.x + idx];
    acc += neg ? -v : v;
  }
  a.part[(size_t)k * a.CG * 64u + c] = live ? acc : 0.0;
}

int discrete_energy(thrml_prog *p, thrml_state *st, double *out) {
  DiscEnergyArgs a;
  a.cat = p->cat_bytes == 1 ? st->cat.as<uint8_t>() : nullptr;
  a.cat16 = p->cat_bytes == 2 ? st->cat.as<uint16_t>() : nullptr;
  a.terms = p->d_terms.as<uint4>();
  a.tsp = p->d_tsp.as<uint32_t>();
  a.W = p->d_w.as<float>();
  a.n_terms = p->d_nterms;
  a.n_ch = std::max<uint32_t>(1u, cdiv32(p->d_nterms, DISC_EN_CHUNK));
  a.C = st->C;
  a.Cp = st->Cp;
  a.CG = (st->C + 63u) / 64u;
  DevBuf part;
  if (int rc = part.alloc((size_t)a.n_ch * a.CG * 64u * sizeof(double))) return rc;
  a.part = part.as<double>();
  const uint64_t waves = (uint64_t)a.n_ch * a.CG;
  hipLaunchKernelGGL(discrete_energy_kernel, dim3(cdiv32(waves, 4)), dim3(256), 0, p->ctx->stream, a);
  THRML_HIP(hipGetLastError());
  return reduce_energy(p, st->C, a.part, a.n_ch, a.CG * 64u, out);
}

}  // namespace thrml
