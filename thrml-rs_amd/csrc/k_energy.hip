// k_energy.hip -- per-chain energies of a device state.
//
// Spin programs: IsingEBM::energy_batched (crates/thrml-models/src/ising.rs:226-320),
//   E[c] = -beta (sum_i b_i s_i + sum_e J_e s_u s_v),  s = 2x - 1,
// over the nodes that have a position in the program's blocks.
// Categorical programs: the sum of DiscreteEBMFactor::factor_energy
// (crates/thrml-models/src/discrete_ebm.rs:551-593) over the program's bias
// factor and edge factor,
//   E[c] = -(sum_n b[n][x_n] + sum_e W[e][x_u][x_v]).
//
// Work split: a wave takes one chunk of edges (or positions) for 64 chains,
// lane = chain.  For spins, s_u s_v = -1 exactly where the two endpoint words
// differ in the lane's bit, so an edge costs three readlanes, a select, a
// conversion and an f64 add per wave.
// Each wave writes one f64 partial per chain; energy_reduce_kernel sums a
// chain's partials in a fixed order, so the result does not depend on the
// schedule (the same state gives the same bits on every call).
#include <algorithm>
#include <mutex>

#include "dev_util.hpp"
#include "internal.hpp"

namespace thrml {

constexpr uint32_t EN_CHUNK_CAT = 128;  // categorical programs: edges or positions per wave

struct SpinEnergyArgs {
  const uint64_t *words;  // state words, group 0
  uint64_t plane_stride;
  const uint2 *epos;      // [n_e] endpoint positions of the edges
  const float *ew;        // [n_e] J_e
  const float *bias;      // [n_pos] b of the node at each position
  uint64_t n_e, n_pos;
  uint32_t n_ech, n_bch;  // edge chunks, position chunks
  uint32_t chunk;         // edges or positions per chunk (a multiple of 64)
  uint32_t G;
  double *part;           // [n_ech + n_bch][G * 64]
};

__global__ __launch_bounds__(256) void spin_energy_kernel(SpinEnergyArgs a) {
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t n_ch = a.n_ech + a.n_bch;
  const uint32_t task = blockIdx.x * 4u + wave;
  if (task >= n_ch * a.G) return;
  const uint32_t g = task / n_ch, k = task - g * n_ch;
  const uint64_t *w = a.words + (size_t)g * a.plane_stride;
  const bool edges = k < a.n_ech;
  const uint64_t i0 = (uint64_t)(edges ? k : k - a.n_ech) * a.chunk;
  const uint64_t i1 = std::min<uint64_t>(i0 + a.chunk, edges ? a.n_e : a.n_pos);
  double acc = 0.0;
  // 64 edges (positions) at a time: lane j loads item i + j with coalesced
  // loads and gathers its words; each item's word and weight then reach every
  // lane by readlane.  Missing items have weight 0 (a +-0 term).
  for (uint64_t i = i0; i < i1; i += 64u) {
    const uint64_t it = i + lane;
    float wt = 0.0f;
    uint64_t x = 0ull;
    if (it < i1) {
      if (edges) {
        const uint2 pp = a.epos[it];
        wt = a.ew[it];
        x = ~(w[pp.x] ^ w[pp.y]);  // bit set: s_u s_v = +1
      } else {
        wt = a.bias[it];
        x = w[it];                 // bit set: s = +1
      }
    }
    const uint32_t xlo = (uint32_t)x, xhi = (uint32_t)(x >> 32);
    const uint32_t wb = __builtin_bit_cast(uint32_t, wt);
    static_for<64>([&](auto j_c) {
      constexpr int j = decltype(j_c)::value;
      // readlane returns a signed int: widen through uint32_t, or a low word
      // with bit 31 set would sign-extend into the high half
      const uint64_t xj = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(xhi, j) << 32) |
                          (uint32_t)__builtin_amdgcn_readlane(xlo, j);
      const float wj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(wb, j));
      acc += (double)(lane_bit(xj) ? wj : -wj);
    });
  }
  a.part[(size_t)k * a.G * 64u + g * 64u + lane] = acc;
}

struct CatEnergyArgs {
  const uint8_t *cat;     // [n_pos][Cp] categories, chains fastest (q <= 256)
  const uint16_t *cat16;  // the same with two bytes per category (q > 256), else null
  const uint2 *epos;      // [n_e] endpoint positions (u role, v role)
  const float *W;         // [E][q][q]
  const float *bias;      // [n_pos][q]
  uint64_t n_e, n_pos;
  uint32_t Cp, C, q, n_ech, n_bch, CG;
  double *part;           // [n_ech + n_bch][CG * 64]
};

__global__ __launch_bounds__(256) void cat_energy_kernel(CatEnergyArgs a) {
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t n_ch = a.n_ech + a.n_bch;
  const uint32_t task = blockIdx.x * 4u + wave;
  if (task >= n_ch * a.CG) return;
  const uint32_t g = task / n_ch, k = task - g * n_ch;
  const uint32_t c = g * 64u + lane;
  const bool live = c < a.C;
  const uint32_t cc = live ? c : 0u;  // dead lanes read chain 0 and add nothing
  const uint32_t qm = a.q - 1u;
  const uint64_t qq = (uint64_t)a.q * a.q;
  auto cat = [&](size_t at) -> uint32_t { return a.cat16 ? a.cat16[at] : a.cat[at]; };
  double acc = 0.0;
  if (k < a.n_ech) {
    const uint64_t e0 = (uint64_t)k * EN_CHUNK_CAT;
    const uint64_t e1 = std::min<uint64_t>(e0 + EN_CHUNK_CAT, a.n_e);
    constexpr uint32_t U = 8;
    uint64_t e = e0;
    for (; e + U <= e1; e += U) {
      uint32_t xu[U], xv[U];
      float v[U];
#pragma unroll
      for (uint32_t i = 0; i < U; ++i) {
        const uint2 pp = a.epos[e + i];
        xu[i] = std::min<uint32_t>(cat((size_t)pp.x * a.Cp + cc), qm);
        xv[i] = std::min<uint32_t>(cat((size_t)pp.y * a.Cp + cc), qm);
      }
#pragma unroll
      for (uint32_t i = 0; i < U; ++i) v[i] = a.W[(e + i) * qq + (uint64_t)xu[i] * a.q + xv[i]];
#pragma unroll
      for (uint32_t i = 0; i < U; ++i) acc += (double)v[i];
    }
    for (; e < e1; ++e) {
      const uint2 pp = a.epos[e];
      const uint32_t x0 = std::min<uint32_t>(cat((size_t)pp.x * a.Cp + cc), qm);
      const uint32_t x1 = std::min<uint32_t>(cat((size_t)pp.y * a.Cp + cc), qm);
      acc += (double)a.W[e * qq + (uint64_t)x0 * a.q + x1];
    }
  } else {
    const uint64_t p0 = (uint64_t)(k - a.n_ech) * EN_CHUNK_CAT;
    const uint64_t p1 = std::min<uint64_t>(p0 + EN_CHUNK_CAT, a.n_pos);
#pragma unroll 8
    for (uint64_t p = p0; p < p1; ++p) {
      const uint32_t x = std::min<uint32_t>(cat((size_t)p * a.Cp + cc), qm);
      acc += (double)a.bias[p * a.q + x];
    }
  }
  a.part[(size_t)k * a.CG * 64u + c] = live ? acc : 0.0;
}

// out[c] = -beta (sum of the position partials + sum of the edge partials) of
// chain c = blockIdx.x, each summed over its rows in a fixed order: thread t
// takes rows t, t + 256, ... (four loads in flight), then a fixed tree.
__global__ __launch_bounds__(256) void energy_reduce_kernel(const double *__restrict__ pe,
                                                            uint32_t ne, uint32_t se,
                                                            const double *__restrict__ pb,
                                                            uint32_t nb, uint32_t sb, double beta,
                                                            double *__restrict__ out) {
  __shared__ double se_[256], sb_[256];
  const uint32_t c = blockIdx.x, t = threadIdx.x;
  double e = 0.0, b = 0.0;
#pragma unroll 4
  for (uint32_t k = t; k < ne; k += 256u) e += pe[(size_t)k * se + c];
#pragma unroll 4
  for (uint32_t k = t; k < nb; k += 256u) b += pb[(size_t)k * sb + c];
  se_[t] = e;
  sb_[t] = b;
  __syncthreads();
  for (uint32_t h = 128u; h > 0u; h >>= 1) {
    if (t < h) {
      se_[t] += se_[t + h];
      sb_[t] += sb_[t + h];
    }
    __syncthreads();
  }
  if (t == 0) out[c] = -beta * (sb_[0] + se_[0]);
}

static inline uint32_t cdiv32(uint64_t x, uint64_t y) { return (uint32_t)((x + y - 1) / y); }

// Device copies of what the energies read and the sweeps do not: endpoint
// positions of every edge whose endpoints both have a position, the raw
// couplings and the raw biases per position.  Built on the first energy call.
static int energy_tables(thrml_prog *p) {
  std::lock_guard<std::mutex> lock(p->en_mu);
  if (p->en_ready) return THRML_OK;
  std::vector<uint32_t> pos;
  std::vector<float> w;
  pos.reserve(2 * p->eu.size());
  if (p->kind != K_POTTS) w.reserve(p->eu.size());
  for (size_t e = 0; e < p->eu.size(); ++e) {
    const int64_t a = p->node_pos[p->eu[e]], b = p->node_pos[p->ev[e]];
    if (a < 0 || b < 0) continue;
    pos.push_back((uint32_t)a);
    pos.push_back((uint32_t)b);
    if (p->kind != K_POTTS) w.push_back(p->w_raw[e]);
  }
  p->en_ne = pos.size() / 2;
  int rc = upload_to(p->ctx, p->en_pos, pos);
  if (!rc && p->kind != K_POTTS) rc = upload_to(p->ctx, p->en_w, w);
  if (!rc && p->kind != K_POTTS) {
    std::vector<float> b(p->n_total);
    for (uint64_t k = 0; k < p->n_total; ++k) b[k] = p->bias_raw[p->pos_node[k]];
    rc = upload_to(p->ctx, p->en_bias, b);
  }
  if (!rc) {
    hipError_t e = hipStreamSynchronize(p->ctx->stream);
    if (e != hipSuccess) rc = hip_fail(e, "energy tables");
  }
  if (rc) return rc;
  p->device_bytes += p->en_pos.bytes + p->en_w.bytes + p->en_bias.bytes;
  p->en_ready = true;
  return THRML_OK;
}

static int finish_energy(thrml_prog *p, uint32_t C, const double *pe, uint32_t ne, uint32_t se,
                         const double *pb, uint32_t nb, uint32_t sb, double beta, double *out) {
  DevBuf dout;
  if (int rc = dout.alloc((size_t)C * sizeof(double))) return rc;
  hipLaunchKernelGGL(energy_reduce_kernel, dim3(C), dim3(256), 0, p->ctx->stream, pe, ne, se, pb,
                     nb, sb, beta, dout.as<double>());
  THRML_HIP(hipGetLastError());
  THRML_HIP(hipMemcpyAsync(out, dout.p, (size_t)C * sizeof(double), hipMemcpyDeviceToHost,
                           p->ctx->stream));
  THRML_HIP(hipStreamSynchronize(p->ctx->stream));
  return THRML_OK;
}

int reduce_energy(thrml_prog *p, uint32_t C, const double *part, uint32_t n, uint32_t stride,
                  double *out) {
  return finish_energy(p, C, part, n, stride, nullptr, 0, stride, 1.0, out);
}

int spin_energy(thrml_prog *p, thrml_state *st, double *out) {
  if (int rc = energy_tables(p)) return rc;
  const bool dense = p->kind == K_DENSE;
  // dense programs: the coupling term comes from the matrix cores
  const uint64_t n_e = dense ? 0 : p->en_ne;
  SpinEnergyArgs a;
  a.words = st->words.as<uint64_t>();
  a.plane_stride = p->n_total;
  a.epos = p->en_pos.as<uint2>();
  a.ew = p->en_w.as<float>();
  a.bias = p->en_bias.as<float>();
  a.n_e = n_e;
  a.n_pos = p->n_total;
  a.G = st->G;
  // 1024 items per wave, or fewer while that leaves under ~2 waves per SIMD
  a.chunk = 1024;
  while (a.chunk > 64 && (cdiv32(n_e, a.chunk) + cdiv32(p->n_total, a.chunk)) * (uint64_t)a.G < 2048)
    a.chunk /= 2;
  a.n_ech = cdiv32(n_e, a.chunk);
  a.n_bch = cdiv32(p->n_total, a.chunk);
  const uint32_t S = st->G * 64u;
  DevBuf part, dpart;
  if (int rc = part.alloc((size_t)(a.n_ech + a.n_bch) * S * sizeof(double))) return rc;
  a.part = part.as<double>();
  const uint64_t waves = (uint64_t)(a.n_ech + a.n_bch) * st->G;
  hipLaunchKernelGGL(spin_energy_kernel, dim3(cdiv32(waves, 4)), dim3(256), 0, p->ctx->stream, a);
  THRML_HIP(hipGetLastError());
  const double *pe = a.part;
  uint32_t ne = a.n_ech, se = S;
  if (dense) {
    // keep the visible operand bits in step with the state words, then the
    // coupling term per (32 hidden sites, chain)
    if (int rc = launch_dense_sync_act(st, 0)) return rc;
    if (int rc = dpart.alloc((size_t)(p->Hp / 32u) * st->C_pad * sizeof(double))) return rc;
    if (int rc = launch_dense_energy(p, st, dpart.as<double>())) return rc;
    pe = dpart.as<double>();
    ne = p->Hp / 32u;
    se = st->C_pad;
  }
  return finish_energy(p, st->C, pe, ne, se, a.part + (size_t)a.n_ech * S, a.n_bch, S,
                       (double)p->beta, out);
}

int potts_energy(thrml_prog *p, thrml_state *st, double *out) {
  if (int rc = energy_tables(p)) return rc;
  CatEnergyArgs a;
  a.cat = p->cat_bytes == 1 ? st->cat.as<uint8_t>() : nullptr;
  a.cat16 = p->cat_bytes == 2 ? st->cat.as<uint16_t>() : nullptr;
  a.epos = p->en_pos.as<uint2>();
  a.W = p->wts.as<float>();
  a.bias = p->bias_w.as<float>();
  a.n_e = p->en_ne;
  a.n_pos = p->n_total;
  a.Cp = st->Cp;
  a.C = st->C;
  a.q = p->q;
  a.n_ech = cdiv32(a.n_e, EN_CHUNK_CAT);
  a.n_bch = cdiv32(p->n_total, EN_CHUNK_CAT);
  a.CG = (st->C + 63u) / 64u;
  const uint32_t S = a.CG * 64u;
  DevBuf part;
  if (int rc = part.alloc((size_t)(a.n_ech + a.n_bch) * S * sizeof(double))) return rc;
  a.part = part.as<double>();
  const uint64_t waves = (uint64_t)(a.n_ech + a.n_bch) * a.CG;
  hipLaunchKernelGGL(cat_energy_kernel, dim3(cdiv32(waves, 4)), dim3(256), 0, p->ctx->stream, a);
  THRML_HIP(hipGetLastError());
  return finish_energy(p, st->C, a.part, a.n_ech, S, a.part + (size_t)a.n_ech * S, a.n_bch, S,
                       1.0, out);
}

}  // namespace thrml
