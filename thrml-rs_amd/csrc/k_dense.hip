// k_dense.hip -- dense bipartite (RBM-shaped) Ising half-sweep on the matrix
// cores of gfx950.
//
// The reference has no dense path: an RBM is an IsingEBM whose edges are the
// complete bipartite graph (crates/thrml-models/src/ising.rs:26-143), run as a
// padded-ELL gather of width H / V (crates/thrml-samplers/src/program.rs:114-230).
// Its spin update (crates/thrml-samplers/src/spin_gibbs.rs:56-100,512-637) for
// the hidden block is
//   gamma[c][h] = beta*c_h + sum_v beta*W[v][h] * (2 s_v[c] - 1)
// and symmetrically for the visible block: one GEMM per half-sweep,
//   Gamma^T[site][chain] = A[site][k] * S[chain][k]^T,
// A = W^T (hidden update, k = v) or W (visible update, k = h), S the +-1
// activations of the other block, bf16 operands with f32 accumulation.
//
// Layout: weights as bf16 [Mp][Kp] (k contiguous, zero padded to multiples of
// 128); the other operand as spin-down bits, one bit vector per chain
// ([C_pad][Kp/32] u32, 1/16 of a bf16 copy, so all of it stays in an XCD's L2)
// expanded to +-1 bf16 in registers; the bit-packed state words stay the
// canonical state.
//
// Kernel: a workgroup of 8 waves computes a 128-site x 128-chain tile of
// Gamma^T with v_mfma_f32_32x32x16_bf16 (4 quadrants of 64 x 64 = 2 x 2 MFMA
// tiles, two waves per quadrant splitting K).  64-wide K slices of the
// weights (16 KiB, XOR-swizzled 16-byte chunks) and of the tile's spin bits
// (1 KiB) move by direct-to-LDS loads (global_load_lds_dwordx4 / _dword)
// through a ring of four LDS stages, issued three slices ahead of the MFMAs,
// so no register staging and no per-slice load latency is exposed.
// The epilogue: one v_permlane32_swap per accumulator pair gives every lane
// one chain and the wave's 32 sites, so per 16 sites one ChaCha8
// block of the chain's stream gives the uniforms (site i of the block takes
// keystream word i), u <= sigmoid(2 gamma) decides, a ballot per site forms
// the 64-chain state word, and the lane writes its new spin-down bits for the
// next half-sweep's GEMM.
#include "dev_util.hpp"
#include "internal.hpp"

namespace thrml {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int TM = 128;  // sites per workgroup tile
constexpr int TN = 128;  // chains per workgroup tile
constexpr int TK = 64;   // K slice per LDS stage
constexpr int NS = 4;    // LDS stages in the ring (slices in flight: NS - 1)
constexpr uint32_t A_BYTES = TM * TK * 2;       // weight slice, bf16: 1024 16-byte chunks
constexpr uint32_t D_BYTES = TN * 8;            // spin bits, 2 words per chain
constexpr uint32_t STAGE = A_BYTES + 2 * D_BYTES;  // (+ a second copy of the bits, see below)
constexpr uint32_t DENSE_LDS = NS * STAGE;      // 72 KiB (dynamic)
constexpr uint32_t DMA_PER_STAGE = 3;           // per wave: 2 x 16 B + 1 x 4 B per lane


struct DenseArgs {
  const uint16_t *A;     // [Mp][Kp] bf16 weights of the sites being updated
  const uint32_t *D;     // [C_pad][Kp/32] spin-down bits of the other block
  const float *bias;     // [Mp] fl(beta * b), zero padded
  const uint32_t *keys;  // [G*64][KEY_WORDS]
  uint64_t *words;       // state words of this block, group 0 (stride plane_stride)
  uint32_t *dout;        // [C_pad][Mp/32] new spin-down bits of this block
  double *epart;         // energy mode: [Mp/32][C_pad] coupling-term partials
  uint64_t plane_stride;
  uint32_t M, Mp, Kp, C, G, n_nt;
  float beta;
};

// Direct-to-LDS loads: lane l's 16 (4) bytes from g go to LDS address
// m0 + 16 l (4 l).  Issued from inline assembly so that the compiler does not
// track them: the main loop waits for them with explicit vmcnt values (it
// issues no other vector-memory operation).  M0 written by the SALU needs one
// wait state before an LDS-DMA load reads it.
__device__ __forceinline__ void dma16(const void *g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(g), "s"(lds)
               : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void *g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off"
               :
               : "v"(g), "s"(lds)
               : "memory", "m0");
}

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// Spin-down bits of 32 consecutive positions k0 + i (i = 0..31) in one u32,
// laid out for the MFMA operand: position 8g + 2j + h (group g of 8, pair j,
// half h) sits at bit 16h + 15 - (4g + j).  Shifting the word left by
// 4g + j then puts the pair's two spins at bits 15 and 31, the sign bits of
// the two bf16 halves of operand dword j.
__host__ __device__ constexpr uint32_t dbit_pos(uint32_t i) {
  return ((i & 1u) ? 31u : 15u) - (4u * (i >> 3) + ((i >> 1) & 3u));
}

// The eight spins of one group as the bf16 MFMA operand (+1 = 0x3F80 up,
// -1 = 0xBF80 down; element 2j in the low half of dword j), from a word
// already shifted left by 4g - S, S = 0 or 8 (`S` completes the shift).
template <int S>
__device__ __forceinline__ bf16x8 spins_bf16(uint32_t w) {
  uint4 r;
  r.x = ((w << S) & 0x80008000u) | 0x3F803F80u;
  r.y = ((w << (S + 1)) & 0x80008000u) | 0x3F803F80u;
  r.z = ((w << (S + 2)) & 0x80008000u) | 0x3F803F80u;
  r.w = ((w << (S + 3)) & 0x80008000u) | 0x3F803F80u;
  return __builtin_bit_cast(bf16x8, r);
}

// A workgroup of 8 waves computes one 128 x 128 tile.  Waves w and w + 4
// own the same 64 x 64 quadrant and split every 64-wide K slice between them
// (k steps 0-1 and 2-3), so two waves share each SIMD: one wave's VALU work
// (spin expansion, epilogue) overlaps the other's MFMAs.  At the end the two
// partial sums of each quadrant are exchanged through LDS (wave group g keeps
// row tile g) and each wave runs the epilogue for its 32 sites.
//
// ENERGY: the same product for the current state, with an epilogue that
// forms the coupling term of the energy instead of sampling: lane c adds
// s_site * Gamma^T[site][c] (s = +-1 of the chain at the site, from the state
// words) over the wave's 32 sites in f64 and writes one partial.
template <bool ENERGY>
__global__ __launch_bounds__(512) void dense_half_kernel(DenseArgs a) {
  extern __shared__ __align__(16) uint8_t dlds[];

  const uint32_t tid = threadIdx.x;
  const uint32_t lane = tid & 63u;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t gi = wave >> 2;                  // K half of each slice, later row tile
  const uint32_t wm = (wave >> 1) & 1u, wn = wave & 1u;  // quadrant
  // tiles ordered chains fastest: each XCD's contiguous range covers few
  // weight-row tiles and all chains, which stay in its L2
  const uint32_t tile = xcd_remap(blockIdx.x, gridDim.x);
  const uint32_t m0 = (tile / a.n_nt) * TM;  // first site
  const uint32_t n0 = (tile % a.n_nt) * TN;  // first chain

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // DMA sources.  Weight chunk P = 64 (8t + wave) + lane (t = 0, 1) of a
  // stage holds row r = P / 8, 16-byte column c = (P % 8) ^ (r % 8): the XOR
  // spreads the 32 rows of one MFMA fragment read over all LDS banks.  The
  // stage's 256 spin-bit words ([chain][2]) are loaded by waves 0-3 and,
  // again into a spare copy, by waves 4-7, so that every wave issues the same
  // three loads per stage and waits for the same count.
  const uint32_t kw = a.Kp / 32u;
  const uint16_t *gA[2];
#pragma unroll
  for (uint32_t t = 0; t < 2; ++t) {
    const uint32_t P = (8u * t + wave) * 64u + lane;
    const uint32_t r = P >> 3, c = (P & 7u) ^ (r & 7u);
    gA[t] = a.A + (size_t)(m0 + r) * a.Kp + c * 8u;
  }
  const uint32_t du = (wave & 3u) * 64u + lane;
  const uint32_t *gD = a.D + (size_t)(n0 + (du >> 1)) * kw + (du & 1u);
  const uint32_t lbase = lds_addr(dlds);
  const uint32_t n_k = a.Kp / TK;
#define THRML_ISSUE(slot, slice)                                                       \
  do {                                                                                  \
    const uint32_t sb_ = lbase + (slot) * STAGE;                                        \
    dma16(gA[0] + (size_t)(slice) * TK, sb_ + wave * 1024u);                            \
    dma16(gA[1] + (size_t)(slice) * TK, sb_ + (8u + wave) * 1024u);                     \
    dma4(gD + (size_t)(slice) * 2u, sb_ + A_BYTES + gi * D_BYTES + (wave & 3u) * 256u); \
  } while (0)
#pragma unroll
  for (int sl = 0; sl < NS - 1; ++sl) THRML_ISSUE((uint32_t)sl, min((uint32_t)sl, n_k - 1u));

  // fragment addresses: row wm*64 + 32i + fr, 16-byte column 2 ks + (lane/32)
  const uint32_t fr = lane & 31u, hf = lane >> 5;
  const uint32_t rowA0 = (wm * 64u + fr) * 128u, rowA1 = rowA0 + 32u * 128u;
  // this wave's two k steps: 2 gi and 2 gi + 1, spin-bit word gi
  const uint32_t cx0 = ((4u * gi + hf) ^ (fr & 7u)) * 16u;
  const uint32_t cx1 = ((4u * gi + 2u + hf) ^ (fr & 7u)) * 16u;
  const uint32_t dA = A_BYTES + (wn * 64u + fr) * 8u + gi * 4u;  // this lane's two chains' word
  // lanes 32..63 take groups 1 and 3 of each word: pre-shift their words by 4
  const uint32_t gsh = hf * 4u;

  for (uint32_t it = 0; it < n_k; ++it) {
    // this wave's DMA for slice it has landed (NS - 2 later slices may be in
    // flight); the barrier then covers every wave's part, and every wave has
    // finished reading the slot refilled next
    wait_vmcnt<(NS - 2) * DMA_PER_STAGE>();
    __builtin_amdgcn_s_barrier();
    THRML_ISSUE((it + NS - 1u) % NS, min(it + NS - 1u, n_k - 1u));
    const uint8_t *st = dlds + (it % NS) * STAGE;
    const uint32_t e = *reinterpret_cast<const uint32_t *>(st + dA) << gsh;
    const uint32_t f = *reinterpret_cast<const uint32_t *>(st + dA + 256u) << gsh;
    bf16x8 fa[2], fn[2], fb[2];
    fa[0] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(st + rowA0 + cx0));
    fa[1] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(st + rowA1 + cx0));
    fn[0] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(st + rowA0 + cx1));
    fn[1] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(st + rowA1 + cx1));
    // first k step: positions 32 gi + 8 hf .. +7 (group 2 gi... of word gi)
    fb[0] = spins_bf16<0>(e);
    fb[1] = spins_bf16<0>(f);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
    // second k step: positions 32 gi + 16 + 8 hf .. +7
    fb[0] = spins_bf16<8>(e);
    fb[1] = spins_bf16<8>(f);
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fn[i], fb[j], acc[i][j], 0, 0, 0);
  }
#undef THRML_ISSUE
  // the trailing (clamped, unread) slices must land before the LDS is reused
  wait_vmcnt<0>();
  __syncthreads();

  // Exchange the partial sums: wave w writes its sums for the other group's
  // row tile (1 - gi) to its 8 KiB region, [j*16 + r][lane]; after the
  // barrier it adds its partner's (wave w ^ 4) sums for row tile gi.
  {
    float *mine = reinterpret_cast<float *>(dlds) + wave * 2048u + lane;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float v0 = acc[0][j][r], v1 = acc[1][j][r];
        mine[(j * 16 + r) * 64] = gi ? v0 : v1;
      }
  }
  __syncthreads();
  float t0[16], t1[16];  // row tile gi, column tiles 0 and 1, summed over K
  {
    const float *other = reinterpret_cast<const float *>(dlds) + (wave ^ 4u) * 2048u + lane;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float a0 = acc[0][0][r], a1 = acc[1][0][r], b0 = acc[0][1][r], b1 = acc[1][1][r];
      t0[r] = (gi ? a1 : a0) + other[r * 64];
      t1[r] = (gi ? b1 : b0) + other[(16 + r) * 64];
    }
  }

  // Epilogue.  MFMA tile (i, j) gives lane l chain j*32 + l%32 and sites
  // i*32 + 8(r/4) + 4(l/32) + r%4.  Swapping the upper half of tile (gi,0)
  // with the lower half of tile (gi,1) leaves every lane l with chain l of
  // the quadrant: lo[r] at site 8(r/4) + r%4, hi[r] at 8(r/4) + 4 + r%4 of
  // row tile gi.
  float lo[16], hi[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, t0[r]),
                                                     __builtin_bit_cast(uint32_t, t1[r]), false, false);
    lo[r] = __builtin_bit_cast(float, (uint32_t)sw[0]);
    hi[r] = __builtin_bit_cast(float, (uint32_t)sw[1]);
  }

  const uint32_t c = n0 + wn * 64u + lane;  // this lane's chain
  const uint32_t g = (n0 >> 6) + wn;        // chain group (wave-uniform)
  if constexpr (ENERGY) {
    const uint32_t sb = m0 + wm * 64u + gi * 32u;
    double e = 0.0;
    if (g < a.G) {  // padded chain groups have no state words
      const uint64_t *wst = a.words + (size_t)g * a.plane_stride;
      static_for<32>([&](auto s_c) {
        constexpr int s = decltype(s_c)::value;
        constexpr int q = s / 8, h = (s / 4) & 1, t = s % 4;
        const float v = h ? hi[4 * q + t] : lo[4 * q + t];
        if (sb + s < a.M) e += (double)(lane_bit(wst[sb + s]) ? v : -v);
      });
    }
    a.epart[(size_t)(sb / 32u) * (a.n_nt * TN) + c] = e;
    return;
  }
  const uint32_t live = g < a.G ? a.C - g * 64u : 0u;
  const uint64_t valid = live >= 64u ? ~0ull : ((1ull << live) - 1ull);
  // the key table holds G*64 chains; padded chains beyond it draw from a zero
  // key (their results are never read)
  uint32_t key[KEY_WORDS];
#pragma unroll
  for (int i = 0; i < KEY_WORDS; ++i) key[i] = 0u;
  if (g < a.G) load_keyx(a.keys, c, key);
  uint64_t *wout = a.words + (size_t)g * a.plane_stride;
  const uint32_t sbase = m0 + wm * 64u + gi * 32u;  // first of this wave's 32 sites
  // lane l < 32 holds the bias of site sbase + l (the bias array is padded to Mp)
  const float bl = a.bias[sbase + (lane & 31u)];
  uint32_t down = 0u;  // spin-down bits of the 32 sites
  static_for<2>([&](auto seg_c) {
    constexpr int seg = decltype(seg_c)::value;
    const uint32_t s0 = sbase + seg * 16u;
    if (s0 < a.M) {
      uint32_t x[16];
      chacha_block_pre<8>(key, s0 >> 4, x);
      uint32_t wlo = 0u, whi = 0u;
      static_for<16>([&](auto k_c) {
        constexpr int k = decltype(k_c)::value;
        constexpr int s = seg * 16 + k;  // site within the row tile
        constexpr int q = s / 8, h = (s / 4) & 1, t = s % 4;
        const float v = h ? hi[4 * q + t] : lo[4 * q + t];
        const uint32_t site = s0 + k;
        const float bk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(uint32_t, bl), s));
        bool up = false;
        if (site < a.M) up = spin_decision(bk + a.beta * v, x[k]);
        const uint64_t mk = __builtin_amdgcn_ballot_w64(up) & valid;
        wlo = writelane<k>(wlo, (uint32_t)mk);
        whi = writelane<k>(whi, (uint32_t)(mk >> 32));
        down |= (up ? 0u : 1u) << dbit_pos(s);
      });
      if (g < a.G && lane < 16u && s0 + lane < a.M) wout[s0 + lane] = ((uint64_t)whi << 32) | wlo;
    }
  });
  a.dout[(size_t)c * (a.Mp / 32u) + sbase / 32u] = down;
}

// Spin-down bits of block b for every chain from the state words (bit order
// dbit_pos); padded positions and chains read as up.
__global__ void dense_sync_bits_kernel(const uint64_t *__restrict__ words, uint64_t plane_stride,
                                       uint32_t G, uint32_t K, uint32_t kw, uint32_t C_pad,
                                       uint32_t *__restrict__ bits) {
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (uint64_t)C_pad * kw) return;
  const uint32_t c = (uint32_t)(t / kw), q = (uint32_t)(t - (uint64_t)c * kw);
  const uint32_t g = c >> 6;
  uint32_t v = 0u;
  if (g < G) {
    for (uint32_t i = 0; i < 32u; ++i) {
      const uint32_t k = q * 32u + i;
      if (k < K && !((words[(size_t)g * plane_stride + k] >> (c & 63u)) & 1ull)) v |= 1u << dbit_pos(i);
    }
  }
  bits[t] = v;
}

static inline uint32_t cdiv_u(uint64_t x, uint64_t y) { return (uint32_t)((x + y - 1) / y); }

int launch_dense_sync_act(thrml_state *st, uint32_t b) {
  thrml_prog *p = st->prog;
  const uint32_t K = b == 0 ? p->V : p->H, Kp = b == 0 ? p->Vp : p->Hp;
  DevBuf &bits = b == 0 ? st->dbits_v : st->dbits_h;
  const uint64_t n = (uint64_t)st->C_pad * (Kp / 32u);
  hipLaunchKernelGGL(dense_sync_bits_kernel, dim3(cdiv_u(n, 256)), dim3(256), 0, p->ctx->stream,
                     st->words.as<uint64_t>() + p->blk_off[b], (uint64_t)p->n_total, st->G, K,
                     Kp / 32u, st->C_pad, bits.as<uint32_t>());
  THRML_HIP(hipGetLastError());
  return THRML_OK;
}

static int dense_args(thrml_prog *p, thrml_state *st, uint32_t b, const uint32_t *d_keys,
                      DenseArgs &a) {
  const bool vis = b == 0;
  a.A = (vis ? p->w_vh : p->w_hv).as<uint16_t>();
  a.D = (vis ? st->dbits_h : st->dbits_v).as<uint32_t>();
  a.bias = p->dense_bias.as<float>() + (vis ? 0 : p->Vp);
  a.keys = d_keys;
  a.words = st->words.as<uint64_t>() + p->blk_off[b];
  a.dout = (vis ? st->dbits_v : st->dbits_h).as<uint32_t>();
  a.plane_stride = p->n_total;
  a.M = vis ? p->V : p->H;
  a.Mp = vis ? p->Vp : p->Hp;
  a.Kp = vis ? p->Hp : p->Vp;
  a.C = st->C;
  a.G = st->G;
  a.beta = p->beta;
  a.n_nt = st->C_pad / TN;
  a.epart = nullptr;
  if (a.Mp % TM || a.Kp % TK || st->C_pad % TN)
    return fail(THRML_EINVAL, "dense program with unpadded operands");
  return THRML_OK;
}

int launch_dense_half(thrml_prog *p, thrml_state *st, uint32_t b, const uint32_t *d_keys) {
  DenseArgs a;
  if (int rc = dense_args(p, st, b, d_keys, a)) return rc;
  const uint32_t n_wg = (a.Mp / TM) * (st->C_pad / TN);
  hipEvent_t t0 = nullptr;
  if (p->ctx->time_begin(0, &t0)) return THRML_EHIP;
  hipLaunchKernelGGL(dense_half_kernel<false>, dim3(n_wg), dim3(512), DENSE_LDS, p->ctx->stream, a);
  THRML_HIP(hipGetLastError());
  return p->ctx->time_end(0, t0);
}

// The coupling term per (32 hidden sites, chain): the hidden block's product
// (A = W^T, other operand = the visible bits, which the caller keeps in step
// with the state words).
int launch_dense_energy(thrml_prog *p, thrml_state *st, double *part) {
  DenseArgs a;
  if (int rc = dense_args(p, st, 1, nullptr, a)) return rc;
  a.epart = part;
  const uint32_t n_wg = (a.Mp / TM) * (st->C_pad / TN);
  hipLaunchKernelGGL(dense_half_kernel<true>, dim3(n_wg), dim3(512), DENSE_LDS, p->ctx->stream, a);
  THRML_HIP(hipGetLastError());
  return THRML_OK;
}

}  // namespace thrml

using namespace thrml;

// Dense bipartite IsingEBM (crates/thrml-models/src/ising.rs:26-143 with the
// complete bipartite edge list e = v*H + h over (v, V+h)): visible block 0 =
// nodes 0..V-1, hidden block 1 = nodes V..V+H-1.
extern "C" int thrml_rbm_program_create(thrml_ctx *ctx, const thrml_rbm_desc *d, thrml_prog **out) {
  if (!ctx || !d || !out) return fail(THRML_EINVAL, "NULL argument");
  if (d->n_visible == 0 || d->n_hidden == 0)
    return fail(THRML_EINVAL, "Encountered an empty block in BlockSpec");
  if (!d->weights_bf16 || !d->bias_visible || !d->bias_hidden)
    return fail(THRML_EINVAL, "NULL argument");
  THRML_HIP(hipSetDevice(ctx->device));
  // the sweep kernel's LDS ring exceeds the default 64 KiB dynamic limit
  THRML_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&dense_half_kernel<false>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)DENSE_LDS));
  THRML_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&dense_half_kernel<true>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)DENSE_LDS));
  const uint32_t V = d->n_visible, H = d->n_hidden;
  const uint32_t Vp = (V + TM - 1) / TM * TM, Hp = (H + TM - 1) / TM * TM;
  auto *p = new thrml_prog();
  p->ctx = ctx;
  p->kind = K_DENSE;
  p->n_free = 2;
  p->n_clamped = 0;
  p->blk_off = {0, V, (uint64_t)V + H};
  p->n_total = (uint64_t)V + H;
  p->node_pos.resize(p->n_total);
  p->pos_node.resize(p->n_total);
  for (uint64_t k = 0; k < p->n_total; ++k) {
    p->node_pos[k] = (int64_t)k;
    p->pos_node[k] = (uint32_t)k;
  }
  p->V = V;
  p->H = H;
  p->Vp = Vp;
  p->Hp = Hp;
  p->beta = d->beta;
  // raw biases per node (visible then hidden), for the energies
  p->bias_raw.assign(d->bias_visible, d->bias_visible + V);
  p->bias_raw.insert(p->bias_raw.end(), d->bias_hidden, d->bias_hidden + H);
  std::vector<uint16_t> wvh((size_t)Vp * Hp, 0), whv((size_t)Hp * Vp, 0);
  for (uint32_t v = 0; v < V; ++v)
    for (uint32_t h = 0; h < H; ++h) {
      const uint16_t w = d->weights_bf16[(size_t)v * H + h];
      wvh[(size_t)v * Hp + h] = w;
      whv[(size_t)h * Vp + v] = w;
    }
  // fl(beta * b): visible at [0, V), hidden at [Vp, Vp + H), zero padding
  std::vector<float> bias((size_t)Vp + Hp, 0.0f);
  for (uint32_t v = 0; v < V; ++v) bias[v] = d->beta * d->bias_visible[v];
  for (uint32_t h = 0; h < H; ++h) bias[Vp + h] = d->beta * d->bias_hidden[h];
  int rc;
  if ((rc = p->w_vh.alloc(wvh.size() * 2)) || (rc = p->w_hv.alloc(whv.size() * 2)) ||
      (rc = p->dense_bias.alloc(bias.size() * 4))) {
    delete p;
    return rc;
  }
  p->device_bytes = p->w_vh.bytes + p->w_hv.bytes + p->dense_bias.bytes;
  hipError_t e = hipMemcpyAsync(p->w_vh.p, wvh.data(), wvh.size() * 2, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess)
    e = hipMemcpyAsync(p->w_hv.p, whv.data(), whv.size() * 2, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess)
    e = hipMemcpyAsync(p->dense_bias.p, bias.data(), bias.size() * 4, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    delete p;
    return hip_fail(e, "dense program upload");
  }
  p->w_bf16_host.assign(d->weights_bf16, d->weights_bf16 + (size_t)V * H);
  *out = p;
  return THRML_OK;
}

// One half-sweep of block blk with explicit per-chain stream keys
// key8[n_chains][8] (the parity tests' entry point).
extern "C" int thrml_rbm_half_sweep(thrml_prog *p, thrml_state *st, int blk, const uint32_t *key8) {
  if (!p || !st || !key8) return fail(THRML_EINVAL, "NULL argument");
  if (p->kind != K_DENSE) return fail(THRML_EINVAL, "not a dense program");
  if (st->prog != p) return fail(THRML_EINVAL, "state belongs to another program");
  if (blk != 0 && blk != 1) return fail(THRML_EINVAL, "block index out of range");
  THRML_HIP(hipSetDevice(p->ctx->device));
  std::vector<uint32_t> k((size_t)st->G * 64u * KEY_WORDS, 0u);
  for (uint32_t c = 0; c < st->C; ++c) key_expand(key8 + (size_t)c * 8u, &k[(size_t)c * KEY_WORDS]);
  DevBuf dk;
  if (int rc = dk.alloc(k.size() * 4)) return rc;
  THRML_HIP(hipMemcpyAsync(dk.p, k.data(), k.size() * 4, hipMemcpyHostToDevice, p->ctx->stream));
  if (int rc = launch_dense_half(p, st, (uint32_t)blk, dk.as<uint32_t>())) return rc;
  THRML_HIP(hipStreamSynchronize(p->ctx->stream));
  return THRML_OK;
}
