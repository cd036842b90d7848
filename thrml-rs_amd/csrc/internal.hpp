// internal.hpp -- library-internal types of libthrml_hip.so.
//
// Device data layout (HBM):
//   state words  uint64_t [G * P][n_total]   G = ceil(n_chains / 64) chain
//                groups, P = bit planes per node (1 for spins, ceil(log2 q)
//                for categories).  Bit l of word (g*P + b, pos) is bit b of
//                the value of chain 64*g + l at global position pos.  A wave
//                of 64 lanes handles one chain group, lane l = chain 64*g + l,
//                so a node's word is wave-uniform (scalar loads) and the new
//                word of a site is one ballot.
//   positions    the reference's global state order: free blocks then clamped
//                blocks, concatenated (crates/thrml-core/src/blockspec.rs:15-67).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <cmath>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/thrml_hip.h"

namespace thrml {

void set_error(const std::string &msg);
int fail(int code, const std::string &msg);
int hip_fail(hipError_t e, const char *what);

#define THRML_HIP(call)                                   \
  do {                                                    \
    hipError_t e_ = (call);                               \
    if (e_ != hipSuccess) return thrml::hip_fail(e_, #call); \
  } while (0)

enum ProgKind : uint32_t { K_LATTICE = 0, K_CSR = 1, K_POTTS = 2, K_DENSE = 3, K_DISCRETE = 4 };

// A device allocation that frees itself.
struct DevBuf {
  void *p = nullptr;
  size_t bytes = 0;
  DevBuf() = default;
  DevBuf(const DevBuf &) = delete;
  DevBuf &operator=(const DevBuf &) = delete;
  ~DevBuf() { release(); }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    bytes = 0;
  }
  int alloc(size_t n) {
    release();
    if (n == 0) n = 16;
    hipError_t e = hipMalloc(&p, n);
    if (e != hipSuccess) {
      p = nullptr;
      return fail(THRML_ENOMEM, "device allocation of " + std::to_string(n) + " bytes failed: " +
                                    hipGetErrorString(e));
    }
    bytes = n;
    return THRML_OK;
  }
  template <class T>
  T *as() const {
    return reinterpret_cast<T *>(p);
  }
};

struct TimingSlot {
  std::vector<hipEvent_t> ev;  // pairs
  size_t used = 0;
  hipEvent_t span0 = nullptr;  // span mode: recorded before the first launch
  uint64_t span_n = 0;         // span mode: launches since span0
};

}  // namespace thrml

struct thrml_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  bool own_stream = false;
  int timing = 0;  // 0 off, 1 an event pair per launch, 2 one span of launches
  // per kernel class: recorded (start, stop) event pairs
  thrml::TimingSlot slots[2];
  double acc_ms[2] = {0, 0};
  uint64_t acc_n[2] = {0, 0};
  int cu_count = 256;
  // The expanded stream keys of the run in flight, grown as needed and reused
  // by later runs (calls on one context are ordered on its stream).  run_mu
  // serialises the runs of host threads that share the context.
  thrml::DevBuf keys;
  std::mutex run_mu;
  int flush_timing(int k);
  int time_begin(int k, hipEvent_t *start);
  int time_end(int k, hipEvent_t start);
};

struct thrml_prog {
  thrml_ctx *ctx = nullptr;
  uint32_t kind = 0;
  uint32_t n_free = 0, n_clamped = 0;
  uint32_t planes = 1;            // bit planes per node
  uint32_t q = 2;                 // categories (2 for spins)
  std::vector<uint64_t> blk_off;  // [n_free + n_clamped + 1]
  uint64_t n_total = 0;
  std::vector<int64_t> node_pos;  // node -> global position (-1: not in any block)
  std::vector<uint32_t> pos_node;
  // Ising parameters (host copies: hinton init and energies)
  float beta = 1.0f;
  std::vector<float> bias_raw;    // [n_nodes]
  std::vector<uint32_t> eu, ev;
  std::vector<float> w_raw;
  uint64_t device_bytes = 0;

  // --- lattice path: one table row of 16 keystream-word thresholds per free
  // position, indexed by the (left, right, up, down) neighbour bits.
  uint32_t L = 0, half = 0;
  uint32_t parity[2] = {0, 0};    // column parity of block b in row 0
  thrml::DevBuf table;            // [n_free_total][16] u32

  // --- CSR path (Ising and Potts): per free position, slots in reference
  // order.  Ising: slot = {tail position, fl(beta*J)}; Potts: u-role slots
  // then v-role slots, slot = {tail position, edge id}.
  thrml::DevBuf row_off;          // [n_free_total + 1] u32 (Ising) / [n_free_total + 1] u32 (Potts u+v)
  thrml::DevBuf slots;            // [n_slots] uint2
  thrml::DevBuf bias_w;           // Ising: [n_free_total] f32 fl(beta*b); Potts: [n_free_total][q]
  thrml::DevBuf uend;             // Potts: [n_free_total] end of the u-role slots
  thrml::DevBuf wts;              // Potts: [E+1][q][q], W[e][a][b] couples x_u = a, x_v = b (edge E: zeros)
  thrml::DevBuf wts_t;            // Potts: [E+1][q][q] transposes (edge E: zeros)
  thrml::DevBuf pslots;           // Potts: [n_free_total][2*pm] uint2, role-padded slots
  uint32_t pm = 0;                // Potts: padded role width (2 or 4), 0 = unpadded kernel
  uint32_t cat_bytes = 1;         // byte-layout programs: bytes per (position, chain), 2 for q > 256
  uint32_t mean_slots = 0;        // Potts: slots per free position, rounded
  uint64_t n_edges = 0;
  bool intra_block_edges = false;
  // Superblocks (crates/thrml-samplers/src/program.rs:28-64): superblock s
  // holds the free blocks sb_off[s] .. sb_off[s+1]-1, all sampled from the
  // state before it.  A staged block writes its new state into the state's
  // staging buffer, which mirrors positions blk_off[first block of s] ..
  // + stage_width[s] (rows of stage_width[s] positions), and the superblock's
  // staged range is copied into place after its last block.  A block is
  // staged when a later block of its superblock reads the state, or when the
  // program has edges inside a block (it then reads its own positions).
  std::vector<uint32_t> sb_off;       // [n_superblocks + 1]
  std::vector<uint32_t> blk_sb;       // free block -> superblock
  std::vector<uint8_t> staged;        // per free block
  std::vector<uint64_t> stage_width;  // per superblock: positions staged (0: none)
  uint64_t stage_max = 0;             // the largest stage_width
  // Ising CSR: per free block, the most slots in a window of 4, 8, 16, 32
  // sites (windows aligned at multiples of their size)
  std::vector<uint32_t> csr_win[4];
  std::vector<uint32_t> csr_maxdeg;  // largest slot count of a site, per free block

  // --- dense bipartite path.  Side 0 ("visible") holds the rows of W, side 1
  // ("hidden") its columns; dense_side[b] is the side of block b (blocks are
  // free ++ clamped in any order) and side_off[s] the global offset of side s.
  uint32_t V = 0, H = 0, Vp = 0, Hp = 0;  // sizes, padded to multiples of 256 (row tiles and K slices)
  uint32_t dense_side[2] = {0, 1};
  uint64_t side_off[2] = {0, 0};
  // Each weight is the exact sum of dense_pieces bf16 values (1 for weights
  // that are bf16 already, up to 3 for any f32); the pieces of a row follow
  // each other along K, each padded alike, so a row holds pieces * Kp values.
  uint32_t dense_pieces = 1;
  thrml::DevBuf w_vh;             // bf16 [Vp][pieces * Hp] (K = H contiguous)
  thrml::DevBuf w_hv;             // bf16 [Hp][pieces * Vp]
  thrml::DevBuf dense_bias;       // f32 [Vp + Hp] fl(beta*b): visible at 0, hidden at Vp

  // --- general discrete factor programs.  blk_kind[b] is 0 for a block of
  // spin nodes, 1 for categorical nodes.  Per free position (row_off), slots
  // in the reference's order (groups in order, head positions ascending),
  // each a uint4 {weight offset, first categorical tail's position or
  // DISC_NONE, first spin tail in d_sp, n_sp | group start << 8 | axis << 9};
  // axis 0: entry c of the row, 2: x * q + c (a head-U slot points at the
  // transposed copy of its factor's weights, so every categorical head reads
  // q contiguous floats; axis 1, c * q + x, is not produced).  Energy terms:
  // one per factor row whose nodes all have positions, two uint4
  // {weight row, first spin in d_tsp, n_sp, x0 position | DISC_NONE},
  // {x1 position | DISC_NONE, d2, 0, 0}.
  std::vector<uint8_t> blk_kind;
  thrml::DevBuf d_slots, d_sp, d_w, d_terms, d_tsp;
  uint64_t d_nterms = 0;

  // --- energies (built on the first energy call): endpoint positions of
  // the edges whose endpoints both have a position, raw J, raw b per position
  std::mutex en_mu;
  bool en_ready = false;
  uint64_t en_ne = 0;
  thrml::DevBuf en_pos;           // [en_ne] uint2
  thrml::DevBuf en_w;             // [en_ne] f32 (spin programs)
  thrml::DevBuf en_bias;          // [n_total] f32 (spin programs)
};

struct thrml_state {
  thrml_prog *prog = nullptr;
  thrml_ctx *ctx = nullptr;  // the program's context: destroy needs no program
  uint32_t C = 0;     // chains
  uint32_t G = 0;     // chain groups of 64
  thrml::DevBuf words;  // spin programs: [G * planes][n_total] u64
  thrml::DevBuf cat;    // categorical programs: [n_total][Cp] u8, chains fastest
  uint32_t Cp = 0;      // C rounded up to 4
  thrml::DevBuf scratch;// per-block staging for programs with intra-block edges / dense operands
  thrml::DevBuf flag;   // u32: set by the import kernels when a value is out of range
  // CSR spin programs with at most 32 chains and no staged block: [n_total]
  // u32, the low halves of the state words (the high halves are zero).  The
  // sweep kernel gathers neighbour states here, half the footprint of the
  // words, and writes both; each run refreshes it from the words first.
  thrml::DevBuf low;
  // dense path operands: spin-down bits per block, one bit vector per chain
  // (bit k%32 of word k/32 is 1 when the spin at block position k is down)
  uint32_t C_pad = 0;     // chains rounded up to the 256-wide GEMM tile
  thrml::DevBuf dbits_v;  // [C_pad][Vp/32] u32
  thrml::DevBuf dbits_h;  // [C_pad][Hp/32] u32
  uint64_t plane_stride() const { return prog->n_total; }
};

// A moment specification bound to a program (ising_moment_spec +
// MomentAccumulatorObserver::new, crates/thrml-observers/src/moment.rs:52,125-150).
// native: lattice programs count in the sweep kernels' layout (ones per
// global position, diff per block-1 site and direction) and slot1/slot2 map
// the requested nodes/pairs onto those counters; otherwise the moment kernel
// counts per requested entry at the positions npos/ppos.
struct thrml_moments {
  thrml_prog *prog = nullptr;
  thrml_ctx *ctx = nullptr;  // the program's context: destroy needs no program
  bool native = false;
  uint64_t n1 = 0, n2 = 0;      // requested nodes, pairs
  uint64_t len1 = 0, len2 = 0;  // counters
  thrml::DevBuf slot1, slot2;   // native: counter index per requested entry
  thrml::DevBuf npos, ppos;     // generic: positions of nodes / pair endpoints
  thrml::DevBuf cnt1, cnt2;     // u32 counters of the current fold period
  thrml::DevBuf acc1, acc2;     // u64 totals
  thrml::DevBuf out;            // int64 staging for host outputs
};

// A general moment observer (MomentAccumulatorObserver with any spec): row r
// multiplies f(x) over the positions pos[row_off[r] .. row_off[r+1]].
struct thrml_observer {
  thrml_prog *prog = nullptr;
  thrml_ctx *ctx = nullptr;
  uint64_t n_rows = 0;
  bool transform = true;
  double max_row_log2 = 0.0;  // byte states: log2 of the largest |product| a row can take
  thrml::DevBuf row_off;  // [n_rows + 1] u64
  thrml::DevBuf pos;      // positions, u32
  thrml::DevBuf acc;      // [n_rows] int64 sums
};

namespace thrml {
// Allocates buf for v and queues the upload on the context's stream.
template <class T>
int upload_to(thrml_ctx *ctx, DevBuf &buf, const std::vector<T> &v) {
  if (int rc = buf.alloc(v.size() * sizeof(T))) return rc;
  if (!v.empty())
    THRML_HIP(hipMemcpyAsync(buf.p, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice,
                             ctx->stream));
  return THRML_OK;
}

// A dense bipartite program: W[i][j] couples node side_nodes[0][i] with node
// side_nodes[1][j]; block k of the global state is side block_side[k], and
// the first n_free blocks are free.  Node ids lie below n_nodes.
struct DenseSpec {
  uint32_t n_nodes = 0;
  std::vector<uint32_t> side_nodes[2];
  std::vector<float> w;          // [n0][n1]
  std::vector<float> bias;       // [n_nodes] raw biases
  float beta = 1.0f;
  uint32_t block_side[2] = {0, 1};
  uint32_t n_free = 2;
};
int dense_program_create(thrml_ctx *ctx, const DenseSpec &d, thrml_prog **out);
// The bf16 pieces w = p[0] + p[1] + p[2] (exact; unused pieces 0) of an f32
// weight, each the nearest bf16 to what the earlier pieces leave.  Returns the
// number of pieces needed (0..3), or -1 when w is not finite or a nonzero
// piece would be a subnormal bf16 (the sum could then be inexact).
__host__ __device__ int bf16_pieces(float w, uint16_t p[3]);

constexpr uint32_t DISC_NONE = 0xffffffffu;
// Programs whose state is one byte per (position, chain): [n_total][Cp].
inline bool byte_layout(const thrml_prog *p) { return p->kind == K_POTTS || p->kind == K_DISCRETE; }
// Values a block of a byte-layout program accepts: 2 for spins, else q.
inline uint32_t block_q(const thrml_prog *p, uint32_t b) {
  return (p->kind == K_DISCRETE && !p->blk_kind[b]) ? 2u : p->q;
}

// Superblocks: set_superblocks checks offsets[n_sb + 1] over the free blocks
// (n_sb = 0: one superblock per free block); plan_staging then decides which
// blocks write through the staging buffer (needs intra_block_edges).
int set_superblocks(thrml_prog *p, uint32_t n_sb, const uint32_t *offsets);
void plan_staging(thrml_prog *p);
// Where free block b writes its new state: in place (false), or into the
// staging buffer at position offset *off with rows of *width positions.
inline bool stage_target(const thrml_prog *p, uint32_t b, uint64_t *off, uint64_t *width) {
  if (!p->staged[b]) return false;
  const uint32_t s = p->blk_sb[b];
  *off = p->blk_off[b] - p->blk_off[p->sb_off[s]];
  *width = p->stage_width[s];
  return true;
}
// Copies superblock s's staged range into the state (no-op when none).
int commit_superblock(thrml_prog *p, thrml_state *st, uint32_t s);

// kernels (launchers return THRML_OK or an error)
// Key tree of one run: run_blocks (mode 0) or sample_with_observation
// (mode 1) with n_chains chains of the root key.
struct KeyPlan {
  uint64_t root;
  uint32_t C, C_pad, n_blocks, mode;
  uint64_t n_iters;                       // mode 0
  uint64_t n_warmup, n_samples, steps;    // mode 1
};
int launch_key_schedule(thrml_ctx *ctx, const KeyPlan &kp, uint64_t s0, uint32_t n_sweeps,
                        uint32_t *d_keys);
// Moment counters of lattice programs: ones[pos] per global position,
// diff[i*4 + d] per block-local site i of block 1 and neighbour direction d
// (0 left, 1 right, 2 up, 3 down).
struct LatticeMoments {
  uint32_t *ones;
  uint32_t *diff;
};
int launch_lattice_half(thrml_prog *p, thrml_state *st, uint32_t b, const uint32_t *d_keys,
                        const LatticeMoments *mom);
int launch_lattice_moments(thrml_state *st, const LatticeMoments *mom);
int launch_csr_half(thrml_prog *p, thrml_state *st, uint32_t b, const uint32_t *d_keys);
// refreshes st->low from the state words (CSR programs that keep it)
int launch_pack_low(thrml_state *st);
void csr_windows(thrml_prog *p, const std::vector<uint32_t> &row_off);
int launch_potts_half(thrml_prog *p, thrml_state *st, uint32_t b, const uint32_t *d_keys);
int launch_discrete_half(thrml_prog *p, thrml_state *st, uint32_t b, const uint32_t *d_keys);
int discrete_energy(thrml_prog *p, thrml_state *st, double *out);
// out[c] = -(sum over rows k < n of part[k * stride + c]) for the state's chains
int reduce_energy(thrml_prog *p, uint32_t C, const double *part, uint32_t n, uint32_t stride,
                  double *out);
// Dense programs: one half-sweep of side `side` (0 rows of W, 1 columns).
int launch_dense_half(thrml_prog *p, thrml_state *st, uint32_t side, const uint32_t *d_keys);
int launch_lattice_table(thrml_prog *p, const uint32_t *d_dir, const float *d_w, const float *d_bias);
int launch_hinton(thrml_prog *p, thrml_state *st, uint32_t b, const uint32_t *d_key8,
                  const float *d_prob);
// State import of block b from device memory; values out of range (spins
// other than 0/1, categories outside 0..q-1) are stored as 0 and set *d_bad.
int launch_potts_pack(thrml_state *st, uint32_t b, const void *d_src, int dtype, uint32_t *d_bad);
int launch_potts_unpack(thrml_state *st, uint32_t b, void *d_dst, int dtype);
int launch_potts_weights(thrml_ctx *ctx, float *w, float *wt, uint64_t n_edges, uint32_t q,
                         uint64_t n_w);
int launch_pack(thrml_state *st, uint32_t b, const void *d_src, int dtype, uint32_t *d_bad);
int launch_unpack(thrml_state *st, uint32_t b, void *d_dst, int dtype);
int launch_moments(thrml_state *st, const uint32_t *d_npos, uint64_t n1, const uint32_t *d_ppos,
                   uint64_t n2, uint32_t *d_ones, uint32_t *d_diff);
// Dense programs: recompute side `side`'s spin-down operand bits from the
// state words.
int launch_dense_sync_act(thrml_state *st, uint32_t side);
int launch_fold_counts(thrml_ctx *ctx, uint32_t *cnt, uint64_t *acc, uint64_t n);
// Adds one observation of st to obs->acc.
int launch_observe(thrml_state *st, thrml_observer *obs);
int launch_finalize_moments(thrml_ctx *ctx, const uint32_t *cnt1, const uint64_t *acc1,
                            const uint32_t *slot1, uint64_t n1, const uint32_t *cnt2,
                            const uint64_t *acc2, const uint32_t *slot2, uint64_t n2, int64_t cn,
                            int64_t *out1, int64_t *out2);
// Per-chain energies of a state into host out[C] (spin: lattice, CSR and
// dense programs; categorical programs).
int spin_energy(thrml_prog *p, thrml_state *st, double *out);
int potts_energy(thrml_prog *p, thrml_state *st, double *out);
// Dense programs: the coupling term sum_h s_h sum_v W[v][h] s_v of every
// chain, as f64 partials [Hp/32][C_pad] (one per 32 hidden sites and chain).
int launch_dense_energy(thrml_prog *p, thrml_state *st, double *part);
int launch_sigmoid_bernoulli(thrml_ctx *ctx, const float *g, const float *u, float *o, uint64_t n);
int launch_fast_math_check(thrml_ctx *ctx, float out[3]);
// Raises *d_bad if one of the n values at d_src is not a state value 0..q-1.
int launch_import_check(thrml_ctx *ctx, const void *d_src, int dtype, uint64_t n, uint32_t q,
                        uint32_t *d_bad);
// The per-device cached self-check (run at the first call on a device).  With
// ok_out NULL it fails with THRML_EUNSUPPORTED when the bounds do not hold;
// otherwise it reports the values and the verdict.
int fast_math_gate(thrml_ctx *ctx, float *v_out, int *ok_out);
// categories of a categorical node: one byte of state per (position, chain)
constexpr uint32_t POTTS_MAX_Q = 256;       // one byte of state per node
constexpr uint32_t POTTS_WIDE_MAX_Q = 65536;  // Potts programs: two bytes above 256
// Categorical blocks with more than 256 categories run one wave per (site,
// chain) item, the lanes splitting the site's nb = q/16 (+1) keystream
// blocks, when that is the faster of the two kernels by their measured costs
// on MI355X (bias-only blocks, q = 300 .. 16384, 16K .. 1M items per launch):
// the wave kernel about 1.1 ns per item for each keystream block a lane
// takes (ceil(nb / 64)); the lane kernel about 0.021 ns per item and block
// once the launch fills the chip, and no less than about 80 us below that
// (each lane walks its nb blocks in sequence).
constexpr uint32_t POTTS_WAVE_MIN_Q = 257;
inline bool potts_wave_pays(uint32_t q, uint64_t items) {
  const double nb = (double)((q + 30u) / 16u);
  const double t_wave = (double)items * std::ceil(nb / 64.0) * 1.1e-3;  // us
  const double t_lane = std::max(80.0, (double)items * nb * 0.021e-3);
  return q >= POTTS_WAVE_MIN_Q && t_wave < t_lane;
}

constexpr uint32_t BATCH_GATHER_MAX_INDICES = 64;
struct BatchGatherStrides {
  uint32_t s[BATCH_GATHER_MAX_INDICES];
  uint32_t batch_stride;
};
int launch_batch_gather(thrml_ctx *ctx, const float *w, uint64_t n_w, const int32_t *idx,
                        uint64_t batch, uint32_t n_idx, const BatchGatherStrides &st, float *out);
int launch_gumbel_argmax(thrml_ctx *ctx, const float *l, const float *u, int32_t *o, uint64_t n,
                         uint32_t q);
}  // namespace thrml
