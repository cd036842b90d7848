/*
 * thrml_hip.h -- C ABI of the MI355X block-Gibbs sweep library
 * (libthrml_hip.so).
 *
 * This is the drop-in boundary for thrml-rs's sampling path: a `-sys` crate
 * declares these functions with `extern "C"` and the reference's
 * thrml-samplers / thrml-models wrappers call them in place of the Burn
 * tensor ops.  Each entry point cites the reference interface it replaces
 * (paths relative to the thrml-rs repository root).
 *
 * Conventions
 *   - Every function returns THRML_OK (0) or a negative THRML_E* code; the
 *     message of the last failure on the calling thread is returned by
 *     thrml_last_error() (the reference returns Result<_, String>).
 *   - Host arrays passed in are copied; the library owns all device memory.
 *   - A program is immutable after creation (the reference's programs are
 *     used through &self).  Calls that take a state enqueue work on the
 *     context's stream and return when it is enqueued, like Burn ops; results
 *     copied to host memory are complete on return.
 *   - Chains: the reference's sweep is single-chain; a state here holds
 *     n_chains independent chains, chain c keyed by RngKey::split(key,
 *     n_chains)[c] (for n_chains == 1 that is the key itself).
 */
#ifndef THRML_HIP_H
#define THRML_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define THRML_OK 0
#define THRML_EINVAL (-1)      /* invalid argument (Err(String) in the reference) */
#define THRML_EHIP (-2)        /* HIP runtime failure */
#define THRML_ENOMEM (-3)      /* device allocation failed */
#define THRML_EUNSUPPORTED (-4)/* valid for the reference, not supported here */

/* element types for state import/export */
#define THRML_DTYPE_U8 0  /* 0/1 spins, or category index */
#define THRML_DTYPE_F32 1 /* the reference's representation: 0.0/1.0, or category as float */

typedef struct thrml_ctx thrml_ctx;     /* one HIP device + one stream */
typedef struct thrml_prog thrml_prog;   /* compiled program (~ BlockSamplingProgram) */
typedef struct thrml_state thrml_state; /* device state of n_chains chains */

/* ---- library / errors -------------------------------------------------- */
int thrml_version(void);
/* Message of the last error on this thread (crates/thrml-samplers/src/program.rs:93-99
 * style strings). */
const char *thrml_last_error(void);

/* ---- context: replaces init_gpu_device / WgpuDevice
 *      (crates/thrml-core/src/backend.rs:55-71) ---------------------------- */
int thrml_ctx_create(int device_ordinal, thrml_ctx **out);
void thrml_ctx_destroy(thrml_ctx *ctx);
/* Use the caller's HIP stream (hipStream_t) instead of the library's own. */
int thrml_ctx_set_stream(thrml_ctx *ctx, void *hip_stream);
void *thrml_ctx_get_stream(thrml_ctx *ctx);
int thrml_ctx_synchronize(thrml_ctx *ctx);
/* Per-kernel timing with HIP events on the context stream (off by default).
 * kernel: 0 = sweep kernel (lattice/CSR/Potts/dense), 1 = moment kernel.
 * enable: 0 off; 1 an event pair around every launch (each pair adds the
 * markers' own few microseconds); 2 one span, from an event before the first
 * launch to one recorded when the time is read, over the launch count (the
 * average launch-to-launch time, gaps and interleaved kernels included).
 * Changing the mode resets the accumulated times. */
int thrml_ctx_enable_timing(thrml_ctx *ctx, int enable);
int thrml_ctx_kernel_time(thrml_ctx *ctx, int kernel, double *avg_ms, uint64_t *count);

/* ---- RngKey: crates/thrml-samplers/src/rng.rs:20-44 ---------------------- */
/* RngKey(key).split(n) -> out[n] (host, bit-exact). */
int thrml_rng_split(uint64_t key, uint64_t n, uint64_t *out);

/* ---- graph builders: crates/thrml-models/src/graph_utils.rs:177-243,
 *      crates/thrml-examples/src/lib.rs:114-205 --------------------------- */
/* Canonical edge list of make_nearest_neighbor_lattice(side, torus) (side is
 * rounded up to even).  Returns the edge count (u, v may be NULL to count). */
int64_t thrml_lattice_edges(uint32_t side, int torus, uint32_t *u, uint32_t *v);
/* The (upper, lower) checkerboard blocks, ascending node id. */
int thrml_lattice_blocks(uint32_t side, uint32_t *upper, uint32_t *lower);
/* greedy_coloring in ascending node order; returns the colour count. */
int64_t thrml_greedy_coloring(uint32_t n_nodes, uint64_t n_edges, const uint32_t *u,
                              const uint32_t *v, uint32_t *color);
/* get_double_grid (crates/thrml-models/tests/test_train_mnist.rs:37-115):
 * two side x side torus layers, upper node i = i and lower node j =
 * side^2 + j; edges (i, side^2 + i), then per jump d the four torus
 * neighbours j of i at distance d (-row, +row, -col, +col), E = side^2 (1 +
 * 4 n_jumps); visible = the first n_visible entries of 0..side^2 shuffled by
 * rand 0.8.5 StdRng::seed_from_u64(seed).  Returns E; with u, v or visible
 * NULL only the count. */
int64_t thrml_double_grid(uint32_t side_len, const uint32_t *jumps, uint32_t n_jumps,
                          uint32_t n_visible, uint64_t seed, uint32_t *u, uint32_t *v,
                          uint32_t *visible);
/* Erdos-Renyi G(n, p) edge list in ascending (min, max) order from the
 * ChaCha8 stream of seed_from_u64(seed); returns the edge count, or the
 * required capacity when it exceeds cap (u, v untouched). */
int64_t thrml_erdos_renyi(uint32_t n_nodes, double p, uint64_t seed, uint32_t *u,
                          uint32_t *v, uint64_t cap);
/* Gaussian parameters from the ChaCha8 stream of seed_from_u64(seed). */
int thrml_param_normal(uint64_t seed, uint64_t n, double mean, double std, float *out);

/* ---- programs ------------------------------------------------------------ */
/* IsingEBM + IsingSamplingProgram::new
 * (crates/thrml-models/src/ising.rs:26-143, 342-388).  Blocks are given as
 * offsets[n_blocks + 1] into a flat array of node ids.  With n_superblocks =
 * 0 each free block is its own superblock, as IsingSamplingProgram builds it
 * (ising.rs:348-349); otherwise the free blocks are grouped into superblocks
 * (see THRML_SUPERBLOCKS below).
 *
 * Execution path: a 2-colour torus lattice runs on the lattice kernel, any
 * other graph on the CSR kernel, both bit-identical to the reference's slot
 * order.  flags = THRML_ISING_DENSE opts in to the matrix-core kernel for a
 * model whose edges are exactly the complete bipartite graph between its two
 * blocks (free ++ clamped, both with at least THRML_DENSE_MIN_SIDE nodes,
 * each pair once in either orientation; an RBM), with any f32 weights (held
 * exactly as sums of up to three bf16 pieces).  That kernel's f32 summation
 * order differs from the slot order, so its decisions can differ from the
 * reference's where |2 gamma - logit u| < 1e-5 (threshold sites); other
 * models ignore the flag.  Without it every model keeps the slot order. */
#define THRML_ISING_DENSE 2u
#define THRML_DENSE_MIN_SIDE 64u
/* THRML_SUPERBLOCKS: BlockGibbsSpec::new over free superblocks
 * (crates/thrml-samplers/src/program.rs:28-64).  Superblock s holds the free
 * blocks superblock_offsets[s] .. superblock_offsets[s+1]-1 (offsets start at
 * 0, end at n_free_blocks and never decrease; an empty superblock does
 * nothing).  Every block of a superblock is sampled from the state before the
 * superblock and the superblock's new state is written after its last block
 * (sample_blocks, crates/thrml-samplers/src/sampling.rs:39-60).  Block b
 * keeps the stream key sweep_key.split(n_free_blocks)[b].  A program with a
 * superblock of two or more blocks runs on the CSR (Ising) or categorical
 * kernel. */
typedef struct {
  uint32_t n_nodes;
  uint64_t n_edges;
  const uint32_t *edge_u; /* [n_edges] */
  const uint32_t *edge_v; /* [n_edges] */
  const float *biases;    /* [n_nodes] */
  const float *weights;   /* [n_edges] */
  float beta;
  uint32_t n_free_blocks;
  const uint32_t *free_offsets; /* [n_free_blocks + 1] */
  const uint32_t *free_nodes;
  uint32_t n_clamped_blocks;
  const uint32_t *clamped_offsets; /* [n_clamped_blocks + 1] or NULL */
  const uint32_t *clamped_nodes;
  uint32_t flags;                  /* 0 or THRML_ISING_DENSE */
  uint32_t n_superblocks;          /* 0: one superblock per free block */
  const uint32_t *superblock_offsets; /* [n_superblocks + 1] or NULL */
} thrml_ising_desc;
int thrml_ising_program_create(thrml_ctx *ctx, const thrml_ising_desc *desc,
                               thrml_prog **out);

/* FactorSamplingProgram over [CategoricalEBMFactor([all], bias[N,q,1]),
 * CategoricalEBMFactor([U, V], W[E,q,q])] with CategoricalGibbsConditional(q, 0)
 * per free block (crates/thrml-models/src/factor.rs:152-185,
 * crates/thrml-models/src/discrete_ebm.rs:456-548,
 * crates/thrml-samplers/src/softmax.rs:228-271).  The global state is the
 * free blocks then the clamped blocks (crates/thrml-core/src/blockspec.rs:15-67);
 * clamped blocks are read as neighbours and never updated.  Superblocks as
 * THRML_SUPERBLOCKS describes (n_superblocks = 0: one per free block, as in
 * crates/thrml-examples/examples/categorical_sampling.rs:149-152). */
typedef struct {
  uint32_t n_nodes;
  uint32_t q; /* 2..65536: one byte of state per node up to 256, two above (read and
                 sample such states as f32) */
  uint64_t n_edges;
  const uint32_t *edge_u;
  const uint32_t *edge_v;
  const float *weights; /* [n_edges][q][q], W[e][a][b] couples x_u = a, x_v = b */
  const float *biases;  /* [n_nodes][q] */
  uint32_t n_free_blocks;
  const uint32_t *free_offsets;
  const uint32_t *free_nodes;
  uint32_t n_clamped_blocks;
  const uint32_t *clamped_offsets; /* [n_clamped_blocks + 1] or NULL */
  const uint32_t *clamped_nodes;
  uint32_t n_superblocks;          /* 0: one superblock per free block */
  const uint32_t *superblock_offsets; /* [n_superblocks + 1] or NULL */
} thrml_potts_desc;
int thrml_potts_program_create(thrml_ctx *ctx, const thrml_potts_desc *desc,
                               thrml_prog **out);

/* Dense bipartite IsingEBM: visible nodes 0..V-1, hidden V..V+H-1, edges
 * (v, V+h) in order e = v*H + h with weight W[v][h], given either in bf16
 * (weights_bf16) or in f32 (weights_f32, the reference's type; each weight
 * is held exactly as the sum of up to three bf16 pieces, and the product
 * takes one pass over K per piece; THRML_EUNSUPPORTED for a weight that is
 * not finite or whose pieces would be subnormal bf16 values).  Blocks:
 * clamped = THRML_RBM_CLAMP_NONE: visible (block 0) and hidden (block 1),
 * both free; THRML_RBM_CLAMP_VISIBLE: free [hidden] (block 0), clamped
 * [visible] (block 1), the data-clamped positive phase of
 * IsingTrainingSpec (crates/thrml-models/src/ising.rs:412-426);
 * THRML_RBM_CLAMP_HIDDEN: free [visible], clamped [hidden].  The same model as
 * thrml_ising_program_create on the complete bipartite edge list, executed
 * with matrix-core GEMMs. */
#define THRML_RBM_CLAMP_NONE 0u
#define THRML_RBM_CLAMP_VISIBLE 1u
#define THRML_RBM_CLAMP_HIDDEN 2u
typedef struct {
  uint32_t n_visible, n_hidden;
  const uint16_t *weights_bf16; /* [V][H], or NULL when weights_f32 is given */
  const float *bias_visible;    /* [V] */
  const float *bias_hidden;     /* [H] */
  float beta;
  uint32_t clamped;             /* THRML_RBM_CLAMP_* */
  const float *weights_f32;     /* [V][H], or NULL when weights_bf16 is given */
} thrml_rbm_desc;
int thrml_rbm_program_create(thrml_ctx *ctx, const thrml_rbm_desc *desc, thrml_prog **out);

/* DiscreteEBMFactor (crates/thrml-models/src/discrete_ebm.rs:293-359): n_spin
 * spin node groups then n_cat (0..2) categorical node groups of `batch` node
 * ids each (nodes[g * batch + b]), weights [batch][d1][d2]: [b, 1, 1] with
 * spin groups only, [b, q, 1] (any d1 d2 = q) with one categorical group,
 * [b, q, q] with two.  SpinEBMFactor and CategoricalEBMFactor are the cases
 * n_cat = 0 and n_spin = 0. */
/* flags = THRML_FACTOR_SQUARE: SquareDiscreteEBMFactor (discrete_ebm.rs:858-
 * 1013): d1 == d2 is required ("Interaction tensor is not square"), and the
 * interaction groups with equal (tail count, spin tail count) are merged
 * (merge_interaction_groups, :909-986): the two categorical-head groups of a
 * factor with two categorical groups become one group, whose slots are summed
 * together (head group 0's slots first). */
#define THRML_FACTOR_SQUARE 1u
typedef struct {
  uint32_t n_spin_groups, n_cat_groups, batch, d1, d2;
  const uint32_t *nodes;  /* [(n_spin_groups + n_cat_groups) * batch] */
  const float *weights;   /* [batch][d1][d2] */
  uint32_t flags;         /* 0 or THRML_FACTOR_SQUARE */
} thrml_discrete_factor;

/* FactorSamplingProgram (crates/thrml-models/src/factor.rs:126-185) over
 * discrete factors: SpinGibbsConditional on blocks of spin nodes,
 * CategoricalGibbsConditional(q) on blocks of categorical nodes
 * (crates/thrml-samplers/src/spin_gibbs.rs:512-595, softmax.rs:586-710).
 * node_kind[n] = 0 for a spin node, 1 for a categorical node with q
 * categories (2..65536, one q per program; ignored without categorical nodes;
 * one byte of state per node up to 256 categories, two above: read and sample
 * such states as f32);
 * every block holds nodes of one kind.  Interaction groups
 * (to_interaction_groups, discrete_ebm.rs:371-540) and slots follow the
 * reference's order: factors in order, per factor the spin-head group, then
 * one group per categorical head; per head node its slots in ascending head
 * position.  A spin head of a factor with two categorical groups reads its
 * weight row, flattened to q*q entries, at the first categorical tail's
 * category (spin_gibbs.rs:553-575).  Superblocks as THRML_SUPERBLOCKS; keys
 * and per-site keystream words as the Ising (spin blocks) and categorical
 * (categorical blocks) programs.  State values: spins 0/1, categories
 * 0..q-1.  Kind 4 (thrml_prog_info). */
typedef struct {
  uint32_t n_nodes;
  const uint8_t *node_kind;  /* [n_nodes] */
  uint32_t q;
  uint32_t n_factors;
  const thrml_discrete_factor *factors;
  uint32_t n_free_blocks;
  const uint32_t *free_offsets;
  const uint32_t *free_nodes;
  uint32_t n_clamped_blocks;
  const uint32_t *clamped_offsets; /* [n_clamped_blocks + 1] or NULL */
  const uint32_t *clamped_nodes;
  uint32_t n_superblocks;          /* 0: one superblock per free block */
  const uint32_t *superblock_offsets;
} thrml_discrete_desc;
int thrml_discrete_program_create(thrml_ctx *ctx, const thrml_discrete_desc *desc,
                                  thrml_prog **out);

void thrml_prog_destroy(thrml_prog *prog);

typedef struct {
  uint32_t kind;        /* 0 Ising lattice, 1 Ising CSR, 2 Potts, 3 dense bipartite,
                           4 discrete factors */
  uint32_t n_free_blocks;
  uint32_t n_clamped_blocks;
  uint64_t n_total;     /* global state length (free ++ clamped) */
  uint64_t device_bytes;/* parameter/table memory held on the device */
  uint32_t dense_pieces;/* dense programs: bf16 pieces per weight (1..3); else 0 */
} thrml_prog_info;
int thrml_prog_get_info(const thrml_prog *prog, thrml_prog_info *out);
/* Length and global offset of block b (free blocks first, then clamped). */
int thrml_prog_block(const thrml_prog *prog, uint32_t b, uint64_t *offset, uint64_t *len);

/* ---- states -------------------------------------------------------------- */
int thrml_state_create(thrml_prog *prog, uint32_t n_chains, thrml_state **out);
/* Destroying a state (or a moment specification) uses only the context, so it
 * may follow the destruction of its program; every other call on it needs the
 * program alive.  Contexts are destroyed last. */
void thrml_state_destroy(thrml_state *st);
/* Write / read block b as [n_chains][block_len] of dtype (host or device
 * memory).  Free blocks carry the sampled state; clamped blocks carry the
 * clamp values (state_clamp of run_blocks). */
int thrml_state_set_block(thrml_state *st, uint32_t b, const void *src, int dtype,
                          int src_on_device);
int thrml_state_get_block(thrml_state *st, uint32_t b, void *dst, int dtype,
                          int dst_on_device);

/* ---- execution ----------------------------------------------------------- */
/* hinton_init (crates/thrml-models/src/ising.rs:602-673) of every free
 * block: s = (u <= sigmoid(beta*b)); block b takes key.split(n_free)[b]
 * and entry (chain c, site i) the keystream word c*block_len + i. */
int thrml_hinton_init(thrml_prog *prog, uint64_t key, thrml_state *st);

/* run_blocks (crates/thrml-samplers/src/sampling.rs:81-106): n_iters sweeps
 * of every free block, in place. */
int thrml_run_blocks(thrml_prog *prog, uint64_t key, thrml_state *st, uint64_t n_iters);

/* run_blocks without allocating: no counterpart in the reference.  For
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  The same sweeps and
 * results as thrml_run_blocks; the run's expanded stream keys go to a fixed
 * THRML_NOALLOC_KEY_BYTES device array of the library (one per GPU, held
 * until the process ends) instead of the context's growable buffer, and no
 * hipMalloc, hipFree or event is made (the array's address and one event per
 * GPU are set up by thrml_ctx_create).  Rejected with THRML_EINVAL: a state
 * whose one sweep needs more key bytes than the array (n_free_blocks x 64
 * ceil(n_chains / 64) x 96; 16 MiB allow n_free_blocks x chain groups <=
 * 2730), and a context with kernel timing on; THRML_EUNSUPPORTED on device
 * ordinals of 64 and above.  Every call on one GPU shares the array and it
 * keeps the last call's contents.  Calls on one GPU hold a per-GPU lock while
 * they queue their launches, and a call on another stream than the previous
 * call's makes its stream wait for the previous call's work (an event
 * recorded after each call), so contexts sharing a GPU do not overwrite each
 * other's keys.  On a stream under graph capture no event is recorded or
 * waited for: captured calls from different streams must be ordered by the
 * caller. */
#define THRML_NOALLOC_KEY_BYTES (16u << 20)
int thrml_run_blocks_noalloc(thrml_prog *prog, uint64_t key, thrml_state *st, uint64_t n_iters);

/* SamplingSchedule (crates/thrml-samplers/src/schedule.rs:4-20) */
typedef struct {
  uint64_t n_warmup, n_samples, steps_per_sample;
} thrml_schedule;

/* sample_with_observation + MomentAccumulatorObserver as used by
 * estimate_moments (crates/thrml-samplers/src/sampling.rs:178-320,
 * crates/thrml-observers/src/moment.rs:157-237,
 * crates/thrml-models/src/ising.rs:455-505).  Returns exact sums over all
 * chains and observations of t_i (nodes[]) and t_a * t_b (pairs[2k], pairs[2k+1])
 * with t = 2s - 1; the reference's moments are sums / n_samples per chain. */
int thrml_estimate_moments(thrml_prog *prog, uint64_t key, thrml_schedule sched,
                           thrml_state *st, const uint32_t *nodes, uint64_t n_nodes,
                           const uint32_t *pairs, uint64_t n_pairs, int64_t *node_sums,
                           int64_t *pair_sums);

/* The moment specification of estimate_moments, built once and reused:
 * ising_moment_spec(nodes, edges) + MomentAccumulatorObserver::new
 * (crates/thrml-observers/src/moment.rs:52-150).  Nodes and pairs are
 * validated and mapped onto the program's counters here. */
typedef struct thrml_moments thrml_moments;
int thrml_moments_create(thrml_prog *prog, const uint32_t *nodes, uint64_t n_nodes,
                         const uint32_t *pairs, uint64_t n_pairs, thrml_moments **out);
void thrml_moments_destroy(thrml_moments *m);
/* sample_with_observation with that observer (sampling.rs:178-320): the same
 * sums as thrml_estimate_moments.  out_on_device = 1: node_sums / pair_sums
 * are device pointers, written on the context stream (no host sync). */
int thrml_moments_run(thrml_prog *prog, uint64_t key, thrml_schedule sched, thrml_state *st,
                      thrml_moments *m, int64_t *node_sums, int64_t *pair_sums,
                      int out_on_device);

/* MomentAccumulatorObserver::new(moment_spec, transform_to_spin)
 * (crates/thrml-observers/src/moment.rs:52-122, observe :153-231) with a
 * general spec, for every program kind: n_rows node tuples, row r =
 * nodes[row_offsets[r] .. row_offsets[r+1]] (the spec's moment types
 * concatenated by the caller; a row may hold any number of nodes, repeats
 * included).  f(x) = 2x - 1 with transform_to_spin, else x (spins 0/1,
 * categories 0..q-1).  Every node must have a position in the program.
 * Categorical rows are multiplied in int64: a row whose product can exceed
 * 2^62 (prod of 2q - 3, or q - 1, over its categorical nodes) is rejected
 * with THRML_EINVAL. */
typedef struct thrml_observer thrml_observer;
int thrml_observer_create(thrml_prog *prog, const uint64_t *row_offsets, uint64_t n_rows,
                          const uint32_t *nodes, int transform_to_spin, thrml_observer **out);
void thrml_observer_destroy(thrml_observer *obs);
/* sample_with_observation (sampling.rs:178-320) with that observer:
 * sums[r] = sum over chains and observations of prod_{x in row r} f(x),
 * exact in int64 (the reference's carry is f32).  sums_on_device = 1: sums
 * is a device pointer, written on the context stream (no host sync).  With
 * categorical rows, a run whose chains x n_samples x largest row product
 * could reach 2^63 is rejected with THRML_EINVAL. */
int thrml_observer_run(thrml_prog *prog, uint64_t key, thrml_schedule sched, thrml_state *st,
                       thrml_observer *obs, int64_t *sums, int sums_on_device);

/* sample_with_observation (crates/thrml-samplers/src/sampling.rs:178-320)
 * with the caller's observer, the reference's AbstractObserver
 * (crates/thrml-observers/src/observer.rs:9-43): observe(user, iteration,
 * st, hip_stream) is called at each observation point, iteration 0 after the
 * warm-up and 1 .. n_samples - 1 after each further steps_per_sample sweeps,
 * with the chains' state in place on the device and the context's stream
 * (hipStream_t), on which the sweeps before it are queued and those after it
 * will be.  The observer keeps its own carry behind `user`.  It may read the
 * state (thrml_state_get_block per block, into host or device memory) and
 * queue work of its own on that stream (the later sweeps then
 * wait for it), but must not change the state or start a run on the same
 * context: thrml_state_set_block, thrml_hinton_init and every run entry point
 * called from inside it on that context fail with THRML_EINVAL.  A nonzero
 * return stops the run and is returned. */
typedef int (*thrml_observe_fn)(void *user, uint64_t iteration, thrml_state *st, void *hip_stream);
int thrml_sample_with_observer(thrml_prog *prog, uint64_t key, thrml_schedule sched,
                               thrml_state *st, thrml_observe_fn observe, void *user);

/* sample_states (crates/thrml-samplers/src/sampling.rs:128-156) for the
 * whole global state: out[n_samples][n_chains][n_total] u8 (host).  A
 * categorical program with more than 256 categories is refused (THRML_EINVAL):
 * sample it with thrml_sample_states_as and THRML_DTYPE_F32. */
int thrml_sample_states(thrml_prog *prog, uint64_t key, thrml_schedule sched,
                        thrml_state *st, uint8_t *out);
/* The same observations in either dtype: out[n_samples][n_chains][n_total] of
 * u8 or of f32 (host), f32 being the StateObserver's own representation
 * (crates/thrml-observers/src/state_observer.rs:12-50: 0.0/1.0 for spins, the
 * category as a float), which holds every category of every program. */
int thrml_sample_states_as(thrml_prog *prog, uint64_t key, thrml_schedule sched,
                           thrml_state *st, void *out, int dtype);

/* Energy per chain of a spin program's state (lattice, CSR or dense), out[C]
 * f64 on the host: IsingEBM::energy_batched (crates/thrml-models/src/ising.rs:226-320),
 * E[c] = -beta (sum_i b_i s_i + sum_e J_e s_u s_v), s = 2x - 1, over the nodes
 * that have a position in the program's blocks (dense programs: J = the bf16
 * weights).  Computed on the device; partial sums are added in a fixed order,
 * so equal states give equal results. */
int thrml_ising_energy(thrml_prog *prog, thrml_state *st, double *out);

/* Energy per chain of a categorical program's state, out[C] f64 on the host:
 * DiscreteEBMFactor::factor_energy (crates/thrml-models/src/discrete_ebm.rs:551-593)
 * summed over the program's bias and edge factors,
 * E[c] = -(sum_n b[n][x_n] + sum_e W[e][x_u][x_v]). */
int thrml_potts_energy(thrml_prog *prog, thrml_state *st, double *out);

/* Energy per chain of a discrete factor program's state, out[C] f64 on the
 * host: DiscreteEBMFactor::factor_energy (crates/thrml-models/src/discrete_ebm.rs:
 * 551-593) summed over the factors, E[c] = -sum_f sum_b W_f[b][x_0][x_1]
 * prod(2 s - 1) (one categorical group: entry x_0 of the row), over the
 * factor rows whose nodes all have a position; f64 accumulation in a fixed
 * order. */
int thrml_discrete_energy(thrml_prog *prog, thrml_state *st, double *out);

/* ---- dense-path pieces exposed for parity tests ---------------------------
 * One half-sweep of side blk (0 visible = rows of W, 1 hidden) of a dense
 * program with explicit per-chain stream keys key8[n_chains][8] (host, the
 * seed_from_u64 words); the side must be a free block. */
int thrml_rbm_half_sweep(thrml_prog *prog, thrml_state *st, int blk, const uint32_t *key8);

/* ---- kernel-level exports mirroring FusedKernelBackend
 *      (crates/thrml-kernels/src/lib.rs:55-106); device pointers ----------- */
/* out[i] = (u[i] < sigmoid(2*gamma[i])) as f32 (sigmoid_bernoulli/kernel.rs:34-55) */
int thrml_sigmoid_bernoulli(thrml_ctx *ctx, const float *gamma, const float *u, float *out,
                            uint64_t n);
/* out[r] = first argmax_j(logits[r][j] - log(-log(u[r][j]))) (gumbel_argmax/kernel.rs:47-88) */
int thrml_gumbel_argmax(thrml_ctx *ctx, const float *logits, const float *u, int32_t *out,
                        uint64_t n_rows, uint32_t q);
/* out[b] = weights[b * batch_stride + sum_i indices[b][i] * strides[i]] for b < batch
 * (batch_gather_fused, lib.rs:86-106; batch_gather/kernel.rs and forward.rs):
 * indices int32 [batch][n_indices] on the device, strides[n_indices] on the
 * host (n_indices <= 64; the reference takes any count), the index arithmetic
 * in u32 with wrapping as the reference's; a linear index at or past
 * n_weights reads 0.0 (one of the values a bounds-checked read of the
 * reference's buffer may give), so no input makes the kernel leave the array. */
int thrml_batch_gather(thrml_ctx *ctx, const float *weights, uint64_t n_weights,
                       const int32_t *indices, uint64_t batch, uint32_t n_indices,
                       const uint32_t *strides, uint32_t batch_stride, float *out);

/* ---- self-check; no counterpart in the reference ---------------------------
 * Worst-case errors of the hardware-math fast paths of the sweep kernels,
 * which their exact decisions rely on (host output, 3 floats):
 * out[0] = max |fast Gumbel score - exact| over all 2^23 uniforms (the
 * categorical kernel requires <= 4e-6); over every float g in [-40, 40],
 * out[1] = max relative error of the hardware e^(-2g) and out[2] = max
 * relative error of the exact sigmoid(2g), both against double precision
 * (the spin kernels require out[1] + out[2] + 2^-23 < 2^-16). */
int thrml_fast_math_check(thrml_ctx *ctx, float *out);
/* The same check as the library keeps it: run once per device at the first
 * program creation (the program is refused with THRML_EUNSUPPORTED when the
 * bounds above do not hold), then cached.  out: the 3 values; *ok = 1 when
 * they satisfy the bounds (thrml_fast_math_bounds_ok). */
int thrml_fast_math_status(thrml_ctx *ctx, float *out, int *ok);
/* 1 when the 3 values of thrml_fast_math_check satisfy the bounds the sweep
 * kernels assume, else 0 (host only). */
int thrml_fast_math_bounds_ok(const float *v);

#ifdef __cplusplus
}
#endif
#endif /* THRML_HIP_H */
