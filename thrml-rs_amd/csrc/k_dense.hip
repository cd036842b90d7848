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
// Layout: weights as bf16 [Mp][P * Kp] (k contiguous, zero padded to
// multiples of 256): a weight that is not a bf16 is held as the exact sum of
// P = 2 or 3 bf16 pieces, piece j of a row at j * Kp, so the product runs
// over P * Kp values of k against the other operand repeated P times (the
// products of +-1 with a bf16 are exact, so only the f32 accumulation order
// differs from an f32 sum).  The other operand as spin-down bits, one bit
// vector per chain ([C_pad][Kp/32] u32, 1/16 of a bf16 copy, so all of it
// stays in an XCD's L2) expanded to +-1 bf16 in registers; the bit-packed
// state words stay the canonical state.
//
// Kernel: a workgroup of 8 waves computes a 64-site x 256-chain tile of
// Gamma^T with v_mfma_f32_32x32x16_bf16 (4 blocks of 64 sites x 64 chains =
// 2 x 2 MFMA tiles, two waves per block splitting K).  The tile is wide in
// chains because the weights dominate the operand traffic: per K slice it
// moves 8 KiB of weights and 2 KiB of spin bits for 64 x 256 outputs.
// 64-wide K slices of the weights (XOR-swizzled 16-byte chunks) and of the
// tile's spin bits move by direct-to-LDS loads (global_load_lds_dwordx4 /
// _dword) through a ring of four LDS stages, issued three slices ahead of the
// MFMAs, so no register staging and no per-slice load latency is exposed.
// The epilogue: one v_permlane32_swap per accumulator pair gives every lane
// one chain and the wave's 32 sites, so per 16 sites one ChaCha8
// block of the chain's stream gives the uniforms (site i of the block takes
// keystream word i), u <= sigmoid(2 gamma) decides, a ballot per site forms
// the 64-chain state word, and the lane writes its new spin-down bits for the
// next half-sweep's GEMM.
#include <algorithm>
#include <cmath>

#include "dev_util.hpp"
#include "internal.hpp"

namespace thrml {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int TM = 64;   // sites per workgroup tile
constexpr int TN = 256;  // chains per workgroup tile
constexpr int TK = 64;   // K slice per LDS stage
constexpr int NS = 4;    // LDS stages in the ring: 3 slices ahead of the one computed
constexpr uint32_t KPAD = TK * NS;  // K (and M) padding: the main loop is unrolled by NS
constexpr uint32_t A_BYTES = TM * TK * 2;       // weight slice, bf16: 512 16-byte chunks
constexpr uint32_t D_BYTES = TN * 8;            // spin bits, 2 words per chain: 512 words
constexpr uint32_t STAGE = A_BYTES + D_BYTES;   // 10 KiB
constexpr uint32_t XCH_BYTES = 8 * 8192;        // the partial-sum exchange: 8 KiB per wave
constexpr uint32_t DENSE_LDS = NS * STAGE > XCH_BYTES ? NS * STAGE : XCH_BYTES;  // 64 KiB (dynamic)
static_assert((NS - 1) * STAGE <= 65535,
              "fragment reads put the stage offset in the 16-bit LDS offset field");
constexpr uint32_t DMA_PER_STAGE = 2;           // per wave: 1 x 16 B + 1 x 4 B per lane


struct DenseArgs {
  const uint16_t *A;     // [Mp][Ka] bf16 weights of the sites being updated (Ka = P * Kp)
  const uint32_t *D;     // [C_pad][Kp/32] spin-down bits of the other block
  const float *bias;     // [Mp] fl(beta * b), zero padded
  const uint32_t *keys;  // [G*64][KEY_WORDS]
  uint64_t *words;       // state words of this block, group 0 (stride plane_stride)
  uint32_t *dout;        // [C_pad][Mp/32] new spin-down bits of this block
  double *epart;         // energy mode: [Mp/32][C_pad] coupling-term partials
  uint64_t plane_stride;
  uint32_t M, Mp, Kp, Ka, kd, C, G, n_nt;  // kd = Kp / TK: K slices per weight piece
  FastDiv div_nt;         // by n_nt
  float beta;
};

// XOR swizzle of the 16-byte chunks of weight-slice row r (8 chunks of 128
// bytes).  A fragment read serves 16 lanes (16 consecutive rows, one chunk
// each) per pass over the 64 four-byte banks; rows r and r + 1 fall in the
// two halves of the bank space (a row is 128 bytes), so the 8 rows of each
// parity must take 8 distinct chunks: (r >> 1) & 7.
__device__ __forceinline__ uint32_t swz(uint32_t r) { return (r >> 1) & 7u; }

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

// The same with a wave-uniform base address and a 32-bit per-lane byte offset
// (the scalar-base form: advancing the base is scalar arithmetic).
__device__ __forceinline__ void dma16s(const void *base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(off), "s"(base), "s"(lds)
               : "memory", "m0");
}
__device__ __forceinline__ void dma4s(const void *base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
               :
               : "v"(off), "s"(base), "s"(lds)
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

// Bit of site s (0..31 of a wave's sites) as the epilogue's four byte chains
// build it (odd sites of segment 0 -> bits 31..24, odd sites of segment 1 ->
// 23..16, even sites of segment 0 -> 15..8, even of segment 1 -> 7..0, each
// chain high bit first): it must be dbit_pos(s).
constexpr uint32_t chain_pos(uint32_t s) {
  return ((s % 16u) & 1u ? (s < 16u ? 24u : 16u) : (s < 16u ? 8u : 0u)) + 7u - (s % 16u) / 2u;
}
constexpr bool chains_match_dbit_pos() {
  for (uint32_t s = 0; s < 32u; ++s)
    if (chain_pos(s) != dbit_pos(s)) return false;
  return true;
}
static_assert(chains_match_dbit_pos(), "epilogue bit chains disagree with dbit_pos");

// The eight spins of one group g as the bf16 MFMA operand (+1 = 0x3F80 up,
// -1 = 0xBF80 down; element 2j in the low half of dword j) from the spin
// word: dword j is (w << (4g + j)) masked to the two sign bits.  The caller
// passes w already shifted by the lane's part of 4g, so the shifts here are
// constants (B + j).  sign = 0x80008000 and one = 0x3F803F80 are passed in
// registers: a v_and_or_b32 (VOP3) cannot encode a literal, and with
// register operands each dword is one shift and one v_and_or_b32.
template <uint32_t B>
__device__ __forceinline__ bf16x8 spins_bf16(uint32_t w, uint32_t sign, uint32_t one) {
  uint4 r;
  r.x = ((w << B) & sign) | one;
  r.y = ((w << (B + 1u)) & sign) | one;
  r.z = ((w << (B + 2u)) & sign) | one;
  r.w = ((w << (B + 3u)) & sign) | one;
  return __builtin_bit_cast(bf16x8, r);
}

// A workgroup of 8 waves computes one 64 x 256 tile.  Waves w and w + 4
// own the same block of 64 sites x 64 chains (chains 64 (w mod 4) + 0..63)
// and split every 64-wide K slice between them (k steps 0-1 and 2-3), so two
// waves share each SIMD: one wave's VALU work (spin expansion, epilogue)
// overlaps the other's MFMAs.  At the end the two partial sums of each block
// are exchanged through LDS (wave group g keeps sites 32 g + 0..31) and each
// wave runs the epilogue for its 32 sites.
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
  const uint32_t gi = wave >> 2;  // K half of each slice, later the 32 sites kept
  const uint32_t wn = wave & 3u;  // block of 64 chains
  // tiles ordered chains fastest: each XCD's contiguous range covers few
  // weight rows and all chains, which stay in its L2
  const uint32_t tile = xcd_remap(blockIdx.x, gridDim.x);
  const uint32_t tr = fdiv(tile, a.div_nt);
  const uint32_t m0 = tr * TM;                   // first site
  const uint32_t n0 = (tile - tr * a.n_nt) * TN;  // first chain

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // DMA sources.  Weight chunk P = 64 wave + lane of a stage holds row
  // r = P / 8, 16-byte column c = (P % 8) ^ swz(r): the XOR spreads each pass
  // of an MFMA fragment read over all LDS banks.  Spin-bit word P ([chain][2])
  // is word P % 2 of chain P / 2.  Every wave issues the same two loads per
  // stage, so all wait for the same count.  Each load is a wave-uniform base
  // (the tile's rows or chains at the slice) plus a fixed per-lane byte
  // offset.
  const uint32_t kw = a.Kp / 32u;
  const uint32_t P = wave * 64u + lane;
  const uint32_t oA = ((P >> 3) * a.Ka + ((P & 7u) ^ swz(P >> 3)) * 8u) * 2u;
  const uint32_t oD = ((P >> 1) * kw + (P & 1u)) * 4u;
  const uint16_t *bA = a.A + (size_t)m0 * a.Ka;
  const uint32_t *bD = a.D + (size_t)n0 * kw;
  const uint32_t lbase = lds_addr(dlds);
  const uint32_t n_k = a.Ka / TK;  // a multiple of NS
  auto issue = [&](uint32_t slot, uint32_t slice) {
    const uint32_t sb = lbase + slot * STAGE;
    const uint16_t *sA = bA + (size_t)slice * TK;
    dma16s(sA, oA, sb + wave * 1024u);
    // every weight piece multiplies the same spins: slice mod kd (at most
    // three pieces)
    uint32_t ds = slice >= a.kd ? slice - a.kd : slice;
    ds = ds >= a.kd ? ds - a.kd : ds;
    dma4s(bD + (size_t)ds * 2u, oD, sb + A_BYTES + wave * 256u);
  };

  // fragment addresses: row 32i + fr, 16-byte column 2 ks + (lane/32).
  // acc[0] accumulates the 32 sites this wave keeps (i = gi), acc[1] the 32
  // it hands to its partner (i = 1 - gi)
  const uint32_t fr = lane & 31u, hf = lane >> 5;
  const uint32_t rowA0 = (gi * 32u + fr) * 128u;
  const uint32_t rowA1 = ((1u - gi) * 32u + fr) * 128u;
  // this wave's two k steps: 2 gi and 2 gi + 1, spin-bit word gi
  const uint32_t cx0 = ((4u * gi + hf) ^ swz(fr)) * 16u;
  const uint32_t cx1 = ((4u * gi + 2u + hf) ^ swz(fr)) * 16u;
  const uint32_t dA = A_BYTES + (wn * 64u + fr) * 8u + gi * 4u;  // this lane's two chains' word
  // the first (second) k step takes groups 0 and 2 (4 and 6) of the spin
  // word for lanes 0..31 and groups 1 and 3 (5 and 7) for lanes 32..63: the
  // lane's words are pre-shifted by 4 hf, then group 4g' + hf sits at
  // constant shift 4g'
  const uint32_t hs = hf * 4u;
  // (one register operand each: a gfx9 VOP3 reads at most one SGPR)
  uint32_t sign;
  asm("v_mov_b32 %0, 0x80008000" : "=v"(sign));
  const uint32_t one = opaque(0x3F803F80u);

  // A wave's operands of one slice, read from the LDS stage SLOT (a constant:
  // the stage offset is the instruction's immediate).
  struct Frag {
    uint32_t e, f;
    bf16x8 a[2], n[2];
  };
  auto load = [&](Frag &F, auto slot_c) {
    constexpr uint32_t SLOT = decltype(slot_c)::value;
    const uint8_t *st = dlds + SLOT * STAGE;
    F.e = *reinterpret_cast<const uint32_t *>(st + dA);
    F.f = *reinterpret_cast<const uint32_t *>(st + dA + 256u);
    F.a[0] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(st + rowA0 + cx0));
    F.a[1] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(st + rowA1 + cx0));
    F.n[0] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(st + rowA0 + cx1));
    F.n[1] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4 *>(st + rowA1 + cx1));
  };
  // The two k steps of a slice: spin operands (first k step: constant
  // shifts 0..3 of the pre-shifted words, weights F.a; second: 8..11, F.n),
  // then four MFMAs.
  auto spins0 = [&](Frag &F, bf16x8 fb[2]) {
    F.e <<= hs;
    F.f <<= hs;
    fb[0] = spins_bf16<0>(F.e, sign, one);
    fb[1] = spins_bf16<0>(F.f, sign, one);
  };
  auto spins1 = [&](const Frag &F, bf16x8 fb[2]) {
    fb[0] = spins_bf16<8>(F.e, sign, one);
    fb[1] = spins_bf16<8>(F.f, sign, one);
  };
  auto mfma4 = [&](const bf16x8 wa[2], const bf16x8 fb[2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wa[i], fb[j], acc[i][j], 0, 0, 0);
  };

  // Software pipeline: slice s is computed from registers read in the step
  // before, while slice s + 1's operands are read from LDS and slice s + 3
  // is loaded into the stage that held slice s - 1.  Step s: (1) every LDS
  // read this wave has issued has returned (lgkmcnt(0): the reads of slice
  // s - 1's stage, issued two steps ago, included) and this wave's part of
  // slice s + 1 has landed (the loads of slice s + 2 may be in flight);
  // (2) the barrier makes every wave's part of slice s + 1 visible, and no
  // wave has a read of slice s - 1's stage outstanding, so it may be
  // refilled; (3) issue slice s + 3; (4) read slice s + 1; (5) compute slice
  // s.  Slices past the end are clamped to the last one (loaded and read
  // again, never computed), so each step issues exactly DMA_PER_STAGE loads
  // per wave and the wait counts are exact.
  //
  // The two waves that share a SIMD (w and w + 4) take the steps in
  // different orders, so that one issues MFMAs while the other issues loads
  // and spin operands: waves 0-3 run (2)-(5) as written; waves 4-7 form the
  // first k step's operands before the barrier and run its MFMAs right after
  // it, then (3), (4) and the second k step.  Barriers alone would keep the
  // pair in phase, both in the load phase at once with the matrix core idle.
  issue(0u, 0u);
  issue(1u, min(1u, n_k - 1u));
  issue(2u, min(2u, n_k - 1u));
  wait_vmcnt<2 * DMA_PER_STAGE>();
  __builtin_amdgcn_s_barrier();
  Frag F0, F1;
  load(F0, std::integral_constant<uint32_t, 0>{});
  auto main_loop = [&](auto late_c) {
    constexpr bool LATE = decltype(late_c)::value;  // waves 4-7
  for (uint32_t it = 0; it < n_k; it += NS) {
    static_for<NS>([&](auto j_c) {
      constexpr uint32_t j = decltype(j_c)::value;
      // Scheduling fences keep the order barrier, loads, reads, MFMAs: the
      // compiler would otherwise move register-only MFMAs of the next slice
      // up next to the reads they depend on, exposing the LDS latency
      Frag &cur = (j & 1u) ? F1 : F0;
      Frag &nxt = (j & 1u) ? F0 : F1;
      constexpr auto next_slot = std::integral_constant<uint32_t, (j + 1u) % NS>{};
      bf16x8 fb[2];
      __builtin_amdgcn_sched_barrier(0);
      asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
      wait_vmcnt<DMA_PER_STAGE>();
      if constexpr (!LATE) {
        __builtin_amdgcn_s_barrier();
        issue((j + 3u) % NS, min(it + j + 3u, n_k - 1u));
        load(nxt, next_slot);
        __builtin_amdgcn_sched_barrier(0);
        spins0(cur, fb);
        mfma4(cur.a, fb);
        spins1(cur, fb);
        mfma4(cur.n, fb);
      } else {
        spins0(cur, fb);
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_barrier();
        mfma4(cur.a, fb);
        __builtin_amdgcn_sched_barrier(0);
        issue((j + 3u) % NS, min(it + j + 3u, n_k - 1u));
        load(nxt, next_slot);
        __builtin_amdgcn_sched_barrier(0);
        spins1(cur, fb);
        mfma4(cur.n, fb);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
  }
  };
  if (gi == 0u) main_loop(std::false_type{});
  else main_loop(std::true_type{});
  // the trailing (clamped, unread) slices must land before the LDS is reused
  wait_vmcnt<0>();
  __syncthreads();

  // Exchange the partial sums: wave w writes its sums for the other group's
  // 32 sites (acc[1]) to its 8 KiB region, [j*16 + r][lane]; after the
  // barrier it adds its partner's (wave w ^ 4) sums for sites 32 gi + 0..31
  // to acc[0].
  {
    float *mine = reinterpret_cast<float *>(dlds) + wave * 2048u + lane;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) mine[(j * 16 + r) * 64] = acc[1][j][r];
  }
  __syncthreads();
  float t0[16], t1[16];  // sites 32 gi + 0..31, chains 0-31 and 32-63, summed over K
  {
    const float *other = reinterpret_cast<const float *>(dlds) + (wave ^ 4u) * 2048u + lane;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      t0[r] = acc[0][0][r] + other[r * 64];
      t1[r] = acc[0][1][r] + other[(16 + r) * 64];
    }
  }

  // Epilogue.  MFMA tile (i, j) gives lane l chain j*32 + l%32 and sites
  // i*32 + 8(r/4) + 4(l/32) + r%4.  Swapping the upper half of tile (gi,0)
  // with the lower half of tile (gi,1) leaves every lane l with chain l of
  // the block: lo[r] at site 8(r/4) + r%4, hi[r] at 8(r/4) + 4 + r%4 of the
  // wave's 32 sites.
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
  const uint32_t sbase = m0 + gi * 32u;     // first of this wave's 32 sites
  if constexpr (ENERGY) {
    const uint32_t sb = sbase;
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
  // the key table holds G*64 chains; padded chains beyond it draw from
  // chain `lane`'s key (their results are never read)
  uint32_t key[KEY_WORDS];
  load_keyx(a.keys, g < a.G ? c : lane, key);
  uint64_t *wout = a.words + (size_t)g * a.plane_stride;
  // the 32 biases by scalar loads (the array is padded to Mp), beta in a VGPR
  // so that the gamma fma reads one SGPR
  float bias[32];
#pragma unroll
  for (int s = 0; s < 32; ++s) bias[s] = a.bias[sbase + s];
  float beta;
  asm("v_mov_b32 %0, %1" : "=v"(beta) : "s"(a.beta));
  // Spin-down bits of the 32 sites for the next product, bit dbit_pos(s) of
  // site s: odd sites of segment 0 fill bits 31..24, odd sites of segment 1
  // bits 23..16, even sites of segment 0 bits 15..8, even sites of segment 1
  // bits 7..0, each in ascending site order, so four byte chains of shift_in
  // build them.  Sites past M (and segments past M) count as up (bit 0).
  uint32_t dh[2] = {0u, 0u}, dl[2] = {0u, 0u};
  static_for<2>([&](auto seg_c) {
    constexpr int seg = decltype(seg_c)::value;
    const uint32_t s0 = sbase + seg * 16u;
    if (s0 < a.M) {
      uint32_t x[16];
      chacha_block_pre<8>(key, s0 >> 4, x);
      uint32_t wlo = 0u, whi = 0u;
      static_for<16>([&](auto k_c) {
        constexpr int k = decltype(k_c)::value;
        constexpr int s = seg * 16 + k;  // site within the wave's 32
        constexpr int q = s / 8, h = (s / 4) & 1, t = s % 4;
        const float v = h ? hi[4 * q + t] : lo[4 * q + t];
        uint64_t up = ~0ull;
        // gamma = fl(beta b) + beta (sum of the products), one rounding: the
        // matrix-core sum already differs from the slot-order sum, so
        // decisions are compared away from threshold sites
        if (s0 + k < a.M) up = spin_decision_mask(__builtin_fmaf(beta, v, bias[s]), x[k]);
        const uint64_t mk = up & valid;
        wlo = writelane<k>(wlo, (uint32_t)mk);
        whi = writelane<k>(whi, (uint32_t)(mk >> 32));
        if constexpr (k & 1) dh[seg] = shift_in(dh[seg], ~up);
        else dl[seg] = shift_in(dl[seg], ~up);
      });
      if (g < a.G && lane < 16u && s0 + lane < a.M) wout[s0 + lane] = ((uint64_t)whi << 32) | wlo;
    }
  });
  a.dout[(size_t)c * (a.Mp / 32u) + sbase / 32u] =
      (dh[0] << 24) | (dh[1] << 16) | (dl[0] << 8) | dl[1];
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

int launch_dense_sync_act(thrml_state *st, uint32_t side) {
  thrml_prog *p = st->prog;
  const uint32_t K = side == 0 ? p->V : p->H, Kp = side == 0 ? p->Vp : p->Hp;
  DevBuf &bits = side == 0 ? st->dbits_v : st->dbits_h;
  const uint64_t n = (uint64_t)st->C_pad * (Kp / 32u);
  hipLaunchKernelGGL(dense_sync_bits_kernel, dim3(cdiv_u(n, 256)), dim3(256), 0, p->ctx->stream,
                     st->words.as<uint64_t>() + p->side_off[side], (uint64_t)p->n_total, st->G, K,
                     Kp / 32u, st->C_pad, bits.as<uint32_t>());
  THRML_HIP(hipGetLastError());
  return THRML_OK;
}

static int dense_args(thrml_prog *p, thrml_state *st, uint32_t side, const uint32_t *d_keys,
                      DenseArgs &a) {
  const bool vis = side == 0;
  a.A = (vis ? p->w_vh : p->w_hv).as<uint16_t>();
  a.D = (vis ? st->dbits_h : st->dbits_v).as<uint32_t>();
  a.bias = p->dense_bias.as<float>() + (vis ? 0 : p->Vp);
  a.keys = d_keys;
  a.words = st->words.as<uint64_t>() + p->side_off[side];
  a.dout = (vis ? st->dbits_v : st->dbits_h).as<uint32_t>();
  a.plane_stride = p->n_total;
  a.M = vis ? p->V : p->H;
  a.Mp = vis ? p->Vp : p->Hp;
  a.Kp = vis ? p->Hp : p->Vp;
  a.Ka = a.Kp * p->dense_pieces;
  a.kd = a.Kp / TK;
  a.C = st->C;
  a.G = st->G;
  a.beta = p->beta;
  a.n_nt = st->C_pad / TN;
  a.div_nt = make_fastdiv(a.n_nt);
  a.epart = nullptr;
  if (a.Mp % TM || a.Kp % KPAD || st->C_pad % TN || p->dense_pieces < 1 || p->dense_pieces > 3)
    return fail(THRML_EINVAL, "dense program with unpadded operands");
  return THRML_OK;
}

int launch_dense_half(thrml_prog *p, thrml_state *st, uint32_t side, const uint32_t *d_keys) {
  DenseArgs a;
  if (int rc = dense_args(p, st, side, d_keys, a)) return rc;
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

namespace thrml {

__host__ __device__ static uint16_t bf16_nearest(float x) {
  const uint32_t b = fbits(x);
  return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

__host__ __device__ int bf16_pieces(float w, uint16_t p[3]) {
  p[0] = p[1] = p[2] = 0;
  if (!__builtin_isfinite(w)) return -1;
  float rest = w;
  int n = 0;
  for (int j = 0; j < 3; ++j) {
    const uint16_t b = bf16_nearest(rest);
    const float f = __builtin_bit_cast(float, (uint32_t)b << 16);
    if ((b & 0x7FFFu) == 0) break;                       // nothing left
    if ((b & 0x7F80u) == 0 || (b & 0x7F80u) == 0x7F80u) return -1;  // subnormal or overflow
    // rest - f is exact in f32: f is rest rounded to 8 significant bits, so
    // the difference holds at most the 16 bits below them
    const double left = (double)rest - (double)f;
    rest = (float)left;
    if ((double)rest != left) return -1;
    p[j] = b;
    n = j + 1;
  }
  return rest == 0.0f ? n : -1;
}

// The most bf16 pieces any weight needs (out[0], at least 1) and whether a
// weight has no exact three-piece form (out[1] != 0): one atomic per wave.
__global__ void dense_pieces_count_kernel(const float *__restrict__ w, uint64_t n,
                                          uint32_t *__restrict__ out) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  uint32_t k = 1u, bad = 0u;
  if (i < n) {
    uint16_t pc[3];
    const int r = bf16_pieces(w[i], pc);
    if (r < 0) bad = 1u;
    else k = r > 1 ? (uint32_t)r : 1u;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    k = max(k, (uint32_t)__shfl_xor((int)k, off));
    bad |= (uint32_t)__shfl_xor((int)bad, off);
  }
  if ((threadIdx.x & 63u) == 0u) {
    atomicMax(out, k);
    if (bad) atomicOr(out + 1, 1u);
  }
}

// Both weight layouts from W [V][H] (f32), P pieces per weight, zero padding:
// w_vh [Vp][P * Hp] (piece j of row v at j * Hp) and w_hv [Hp][P * Vp].  One
// thread per padded (v, h); every element of both arrays is written.
__global__ void dense_layout_kernel(const float *__restrict__ w, uint32_t V, uint32_t H,
                                    uint32_t Vp, uint32_t Hp, uint32_t P,
                                    uint16_t *__restrict__ wvh, uint16_t *__restrict__ whv) {
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (uint64_t)Vp * Hp) return;
  const uint32_t v = (uint32_t)(t / Hp), h = (uint32_t)(t - (uint64_t)v * Hp);
  uint16_t pc[3] = {0, 0, 0};
  if (v < V && h < H) (void)bf16_pieces(w[(size_t)v * H + h], pc);  // checked beforehand
  for (uint32_t j = 0; j < P; ++j) {
    wvh[(size_t)v * Hp * P + (size_t)j * Hp + h] = pc[j];
    whv[(size_t)h * Vp * P + (size_t)j * Vp + v] = pc[j];
  }
}

// A dense bipartite program (the matrix-core path): blocks, node positions,
// both weight layouts and the scaled biases.  The weights are split into
// bf16 pieces and laid out on the device.
int dense_program_create(thrml_ctx *ctx, const DenseSpec &d, thrml_prog **out) {
  const uint32_t V = (uint32_t)d.side_nodes[0].size(), H = (uint32_t)d.side_nodes[1].size();
  if (V == 0 || H == 0) return fail(THRML_EINVAL, "Encountered an empty block in BlockSpec");
  if (d.w.size() != (size_t)V * H) return fail(THRML_EINVAL, "dense weights have the wrong size");
  if (d.block_side[0] == d.block_side[1] || d.block_side[0] > 1 || d.block_side[1] > 1 ||
      d.n_free < 1 || d.n_free > 2)
    return fail(THRML_EINVAL, "dense program blocks must be the two sides, at least one free");
  THRML_HIP(hipSetDevice(ctx->device));
  if (int rc = fast_math_gate(ctx, nullptr, nullptr)) return rc;
  // the fewest bf16 pieces that hold every weight exactly, found on the device
  DevBuf wraw, cnt;
  if (int rc = upload_to(ctx, wraw, d.w)) return rc;
  if (int rc = cnt.alloc(2 * sizeof(uint32_t))) return rc;
  const uint32_t cnt_init[2] = {1u, 0u};
  THRML_HIP(hipMemcpyAsync(cnt.p, cnt_init, sizeof cnt_init, hipMemcpyHostToDevice, ctx->stream));
  const uint64_t n_w = (uint64_t)V * H;
  if ((n_w + 255) / 256 > 0x7fffffffull) return fail(THRML_EUNSUPPORTED, "too many dense weights");
  hipLaunchKernelGGL(dense_pieces_count_kernel, dim3((uint32_t)((n_w + 255) / 256)), dim3(256), 0,
                     ctx->stream, wraw.as<float>(), n_w, cnt.as<uint32_t>());
  THRML_HIP(hipGetLastError());
  uint32_t cnt_h[2] = {0u, 0u};
  THRML_HIP(hipMemcpyAsync(cnt_h, cnt.p, sizeof cnt_h, hipMemcpyDeviceToHost, ctx->stream));
  THRML_HIP(hipStreamSynchronize(ctx->stream));
  if (cnt_h[1])
    return fail(THRML_EUNSUPPORTED, "a dense weight is not finite or not a sum of three normal bf16 values");
  const uint32_t P = std::min(3u, std::max(1u, cnt_h[0]));
  // the sweep kernel's LDS ring exceeds the default 64 KiB dynamic limit
  THRML_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&dense_half_kernel<false>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)DENSE_LDS));
  THRML_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&dense_half_kernel<true>),
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)DENSE_LDS));
  // padded to KPAD (a multiple of TM): both sides serve as rows and as K
  const uint32_t Vp = (V + KPAD - 1) / KPAD * KPAD, Hp = (H + KPAD - 1) / KPAD * KPAD;
  auto *p = new thrml_prog();
  p->ctx = ctx;
  p->kind = K_DENSE;
  p->n_free = d.n_free;
  p->n_clamped = 2 - d.n_free;
  p->n_total = (uint64_t)V + H;
  p->dense_side[0] = d.block_side[0];
  p->dense_side[1] = d.block_side[1];
  const uint64_t len0 = d.block_side[0] == 0 ? V : H;
  p->blk_off = {0, len0, p->n_total};
  set_superblocks(p, 0, nullptr);  // one superblock per free block, nothing staged
  p->side_off[d.block_side[0]] = 0;
  p->side_off[d.block_side[1]] = len0;
  p->node_pos.assign(d.n_nodes, -1);
  p->pos_node.assign(p->n_total, 0);
  for (uint32_t s = 0; s < 2; ++s)
    for (size_t i = 0; i < d.side_nodes[s].size(); ++i) {
      const uint32_t node = d.side_nodes[s][i];
      if (node >= d.n_nodes) {
        delete p;
        return fail(THRML_EINVAL, "Node not found in global location map");
      }
      if (p->node_pos[node] >= 0) {
        delete p;
        return fail(THRML_EINVAL, "Node appears twice in blocks");
      }
      p->node_pos[node] = (int64_t)(p->side_off[s] + i);
      p->pos_node[p->side_off[s] + i] = node;
    }
  p->V = V;
  p->H = H;
  p->Vp = Vp;
  p->Hp = Hp;
  p->beta = d.beta;
  p->bias_raw = d.bias;  // per node, for hinton_init and the energies
  p->dense_pieces = P;
  // fl(beta * b): side 0 at [0, V), side 1 at [Vp, Vp + H), zero padding
  std::vector<float> bias((size_t)Vp + Hp, 0.0f);
  for (uint32_t v = 0; v < V; ++v) bias[v] = d.beta * d.bias[d.side_nodes[0][v]];
  for (uint32_t h = 0; h < H; ++h) bias[Vp + h] = d.beta * d.bias[d.side_nodes[1][h]];
  // piece j of row r at r * (P * Kp) + j * Kp
  const size_t n_lay = (size_t)Vp * Hp * P;
  int rc;
  if ((rc = p->w_vh.alloc(n_lay * 2)) || (rc = p->w_hv.alloc(n_lay * 2)) ||
      (rc = p->dense_bias.alloc(bias.size() * 4))) {
    delete p;
    return rc;
  }
  p->device_bytes = p->w_vh.bytes + p->w_hv.bytes + p->dense_bias.bytes;
  if (((uint64_t)Vp * Hp + 255) / 256 > 0x7fffffffull) {
    delete p;
    return fail(THRML_EUNSUPPORTED, "too many dense weights");
  }
  hipLaunchKernelGGL(dense_layout_kernel, dim3((uint32_t)(((uint64_t)Vp * Hp + 255) / 256)), dim3(256), 0,
                     ctx->stream, wraw.as<float>(), V, H, Vp, Hp, P, p->w_vh.as<uint16_t>(),
                     p->w_hv.as<uint16_t>());
  hipError_t e = hipGetLastError();
  if (e == hipSuccess)
    e = hipMemcpyAsync(p->dense_bias.p, bias.data(), bias.size() * 4, hipMemcpyHostToDevice, ctx->stream);
  // the launches end before any buffer they use is freed, on every path
  const hipError_t es = hipStreamSynchronize(ctx->stream);
  if (e == hipSuccess) e = es;
  if (e != hipSuccess) {
    delete p;
    return hip_fail(e, "dense program upload");
  }
  *out = p;
  return THRML_OK;
}

}  // namespace thrml

// Dense bipartite IsingEBM (crates/thrml-models/src/ising.rs:26-143 with the
// complete bipartite edge list e = v*H + h over (v, V+h)): visible nodes
// 0..V-1, hidden nodes V..V+H-1; blocks [visible, hidden] both free, or the
// free side then the clamped side.
extern "C" int thrml_rbm_program_create(thrml_ctx *ctx, const thrml_rbm_desc *d, thrml_prog **out) {
  if (!ctx || !d || !out) return fail(THRML_EINVAL, "NULL argument");
  if (d->n_visible == 0 || d->n_hidden == 0)
    return fail(THRML_EINVAL, "Encountered an empty block in BlockSpec");
  if (!d->bias_visible || !d->bias_hidden || (!d->weights_bf16) == (!d->weights_f32))
    return fail(THRML_EINVAL, "NULL argument (exactly one of weights_bf16 and weights_f32 is given)");
  if (d->clamped > THRML_RBM_CLAMP_HIDDEN) return fail(THRML_EINVAL, "unknown clamped side");
  const uint32_t V = d->n_visible, H = d->n_hidden;
  if ((uint64_t)V + H > 0xffffffffull) return fail(THRML_EUNSUPPORTED, "more than 2^32-1 nodes");
  DenseSpec s;
  s.n_nodes = V + H;
  s.side_nodes[0].resize(V);
  s.side_nodes[1].resize(H);
  for (uint32_t v = 0; v < V; ++v) s.side_nodes[0][v] = v;
  for (uint32_t h = 0; h < H; ++h) s.side_nodes[1][h] = V + h;
  s.w.resize((size_t)V * H);
  if (d->weights_f32)
    s.w.assign(d->weights_f32, d->weights_f32 + (size_t)V * H);
  else
    for (size_t e = 0; e < s.w.size(); ++e)
      s.w[e] = __builtin_bit_cast(float, (uint32_t)d->weights_bf16[e] << 16);
  s.bias.assign(d->bias_visible, d->bias_visible + V);
  s.bias.insert(s.bias.end(), d->bias_hidden, d->bias_hidden + H);
  s.beta = d->beta;
  s.n_free = d->clamped == THRML_RBM_CLAMP_NONE ? 2u : 1u;
  if (d->clamped == THRML_RBM_CLAMP_VISIBLE) {  // free [hidden], clamped [visible]
    s.block_side[0] = 1;
    s.block_side[1] = 0;
  }
  return dense_program_create(ctx, s, out);
}

// One half-sweep of side blk (0 visible, 1 hidden) with explicit per-chain
// stream keys key8[n_chains][8] (the parity tests' entry point).
extern "C" int thrml_rbm_half_sweep(thrml_prog *p, thrml_state *st, int blk, const uint32_t *key8) {
  if (!p || !st || !key8) return fail(THRML_EINVAL, "NULL argument");
  if (p->kind != K_DENSE) return fail(THRML_EINVAL, "not a dense program");
  if (st->prog != p) return fail(THRML_EINVAL, "state belongs to another program");
  if (blk != 0 && blk != 1) return fail(THRML_EINVAL, "block index out of range");
  bool free_side = false;
  for (uint32_t b = 0; b < p->n_free; ++b) free_side |= p->dense_side[b] == (uint32_t)blk;
  if (!free_side) return fail(THRML_EINVAL, "that side is a clamped block");
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
