/*
 * thrml_oracle.h -- CPU restatement of thrml-rs's block Gibbs sweep.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP product
 * path: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it.  The product never links, imports or calls anything here.
 *
 * Every function follows a named reference file:line (paths relative to the
 * thrml-rs repository root).  The build-defined conventions that the reference
 * leaves open (the per-site uniform stream, the sigmoid / log implementation,
 * the canonical edge order) are restated here independently of the product
 * sources so that a mistake in one is caught by the other.
 *
 * State representation (the reference's own): one byte per node per chain,
 * value 0/1 for spins (crates/thrml-models/src/ising.rs:160 maps it to 2s-1),
 * a category index for categorical nodes.  A chain's state is the global state
 * vector of crates/thrml-core/src/blockspec.rs:15-67: the free blocks then the
 * clamped blocks, concatenated in block order.  `C` chains are stored as
 * state[c * n_total + pos].
 */
#ifndef THRML_ORACLE_H
#define THRML_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* categories of a categorical node: states hold uint16_t per node */
#define ORC_MAX_Q 65536u        /* categorical nodes of discrete factor programs */
#define ORC_POTTS_MAX_Q 65536u  /* categorical (Potts) programs */

/* ---- random numbers: crates/thrml-samplers/src/rng.rs:10-44 ------------- */
/* ChaCha block function, `rounds` = 8 for ChaCha8, 20 for RFC 8439 checks.
 * State words 12,13 = 64-bit block counter, 14,15 = 64-bit stream id. */
void orc_chacha_block(const uint32_t key[8], uint64_t counter, uint64_t stream,
                      int rounds, uint32_t out[16]);
/* rand_core 0.6 SeedableRng::seed_from_u64: PCG32 output fills the seed.
 * Pinned by one remembered rand_core value (seed_from_u64(0)); other seeds
 * take the same restated PCG32 steps. */
void orc_seed_from_u64(uint64_t seed, uint32_t key_out[8]);
/* RngKey::split (rng.rs:20-38): n=0 -> nothing, n=1 -> [key], else n x next_u64
 * of ChaCha8Rng::seed_from_u64(key).  The split semantics are pinned by the
 * reference's tests (rng.rs:57-86); the u64 composition of next_u64
 * (rand_chacha 0.3.1 BlockRng: word 2j | word 2j+1 << 32) is parity unpinned:
 * no crate source, binary or reference-held vector fixes it offline. */
void orc_rng_split(uint64_t key, size_t n, uint64_t *out);
/* A checked copy of superblock offsets over n_free blocks (the identity
 * partition when n_sb = 0); NULL with err filled when invalid. */
uint32_t *orc_sb_partition(uint32_t n_free, uint32_t n_sb, const uint32_t *off,
                           uint32_t *n_out, char *err, size_t errlen);
/* Word w of the ChaCha8 keystream with the given expanded key. */
uint32_t orc_stream_word(const uint32_t key8[8], uint64_t w);

/* ---- decision math (build convention shared with the GPU path) ---------- */
float orc_exp(float x);
float orc_sigmoid(float x);          /* 1 / (1 + exp(-x)), x clamped to [-80,80] */
float orc_log(float x);              /* natural log for x in (0, 1] */
float orc_gumbel(uint32_t word);     /* -log(-log(u)), u = ((w>>8)|1)/2^24 */
/* vectorised: fn 0 = exp, 1 = sigmoid, 2 = log */
/* Full-range forms for arbitrary float inputs (IEEE limits at 0, inf, NaN,
 * subnormals); equal to the three above on their ranges. */
float orc_exp_full(float x);
float orc_sigmoid_full(float x);
float orc_log_full(float x);
/* The reference's kernel-level Gumbel-argmax and sigmoid-Bernoulli
 * (crates/thrml-kernels/src/gumbel_argmax/kernel.rs:47-88,
 * crates/thrml-kernels/src/sigmoid_bernoulli/kernel.rs:34-55) over the
 * full-range math: out[r] = first argmax_k of logits[r][k] + (0 - log(0 -
 * log u[r][k])) under '>', out[i] = (u[i] < 1 / (1 + exp(0 - 2 gamma[i]))). */
void orc_gumbel_argmax(const float *logits, const float *u, int32_t *out, size_t n, uint32_t q);
void orc_sigmoid_bernoulli(const float *gamma, const float *u, float *out, size_t n);
/* batch_gather_fused (crates/thrml-kernels/src/batch_gather/kernel.rs) */
void orc_batch_gather(const float *w, uint64_t n_w, const int32_t *idx, uint64_t batch,
                      uint32_t n, const uint32_t *strides, uint32_t batch_stride, float *out);
/* fn: 0 exp, 1 sigmoid, 2 log, 3 exp_full, 4 sigmoid_full, 5 log_full */
void orc_map_f32(int fn, const float *x, float *y, size_t n);
void orc_map_gumbel(const uint32_t *w, float *y, size_t n);

/* ---- graphs: crates/thrml-models/src/graph_utils.rs:177-243,
 *              crates/thrml-examples/src/lib.rs:114-205 ------------------- */
/* Canonical edge list of the side x side lattice (side rounded up to even).
 * Returns the edge count; u/v may be NULL to only count. */
size_t orc_lattice_edges(uint32_t side, int torus, uint32_t *u, uint32_t *v);
/* upper block = nodes with (i+j) even, lower = odd, ascending node id. */
void orc_lattice_blocks(uint32_t side, uint32_t *upper, uint32_t *lower);
/* Greedy colouring in ascending node order; returns number of colours. */
uint32_t orc_greedy_coloring(uint32_t n, size_t n_edges, const uint32_t *u,
                             const uint32_t *v, uint32_t *color);
/* Gaussian parameters from the ChaCha8 stream of seed_from_u64(seed),
 * Box-Muller in double precision, rounded to f32. */
void orc_param_normal(uint64_t seed, size_t n, double mean, double std, float *out);

/* ---- schedule: crates/thrml-samplers/src/schedule.rs:4-20 ---------------- */
typedef struct {
  uint64_t n_warmup, n_samples, steps_per_sample;
} orc_schedule;

/* ---- Ising program: ising.rs:105-143,342-388; program.rs:88-318 --------- */
typedef struct orc_ising orc_ising;

/* Blocks are given as offsets[n_blocks+1] into a flat node-id array.
 * Returns NULL and fills err on invalid input (messages mirror the
 * reference's error strings). */
orc_ising *orc_ising_create(uint32_t n_nodes, size_t n_edges, const uint32_t *eu,
                            const uint32_t *ev, const float *bias,
                            const float *weight, float beta, uint32_t n_free,
                            const uint32_t *free_off, const uint32_t *free_nodes,
                            uint32_t n_clamped, const uint32_t *clamp_off,
                            const uint32_t *clamp_nodes, char *err, size_t errlen);
void orc_ising_destroy(orc_ising *p);
/* Groups the free blocks into superblocks (BlockGibbsSpec::new,
 * program.rs:28-64): superblock s = free blocks off[s] .. off[s+1]-1; every
 * block of a superblock is sampled from the state before it and the
 * superblock's new state is written after its last block (sample_blocks,
 * sampling.rs:39-60); block b keeps the key sweep_key.split(n_free)[b].
 * n_sb = 0 restores one superblock per free block (the default).  Returns 0,
 * or -1 with err filled. */
int orc_ising_set_superblocks(orc_ising *p, uint32_t n_sb, const uint32_t *off, char *err,
                              size_t errlen);
size_t orc_ising_total(const orc_ising *p);
/* global position of a node, or -1 */
int64_t orc_ising_pos(const orc_ising *p, uint32_t node);

/* hinton_init (ising.rs:602-673) over the free blocks of the program. */
void orc_hinton_init(const orc_ising *p, uint64_t key, uint32_t n_chains,
                     uint8_t *state);
/* run_blocks (sampling.rs:81-106), chain c keyed by RngKey::split(key, C)[c].
 * thr_sites (may be NULL) receives the number of updates whose
 * |2*gamma - logit(u)| < 1e-5. */
void orc_run_blocks(const orc_ising *p, uint64_t key, uint32_t n_chains,
                    uint8_t *state, uint64_t n_iters, int n_threads,
                    uint64_t *thr_sites);
/* sample_with_observation + MomentAccumulatorObserver (sampling.rs:178-320,
 * moment.rs:157-237, ising.rs:455-505).  Sums of t_i and t_i*t_j with t=2s-1
 * over chains and observations, exact in int64. */
void orc_estimate_moments(const orc_ising *p, uint64_t key, orc_schedule sched,
                          uint32_t n_chains, uint8_t *state,
                          const uint32_t *nodes, size_t n1,
                          const uint32_t *pairs, size_t n2, int64_t *node_sums,
                          int64_t *edge_sums, int n_threads, uint64_t *thr_sites);
/* sample_states with every node observed (sampling.rs:128-156): the global
 * state after the warmup and after each later sample, out[n_obs][C][n_total],
 * n_obs = max(n_samples, 1). */
void orc_sample_states(const orc_ising *p, uint64_t key, orc_schedule sched,
                       uint32_t n_chains, uint8_t *state, uint8_t *out, int n_threads);
/* Chains `chains[k]` (k < n_sel) of a C_total-chain run, keyed by
 * RngKey::split(key, C_total)[chains[k]]; state is [n_sel][n_total]. */
void orc_run_blocks_subset(const orc_ising *p, uint64_t key, uint32_t C_total,
                           const uint32_t *chains, uint32_t n_sel, uint8_t *state,
                           uint64_t n_iters, int n_threads);
/* gamma of every free position for one chain's global state (out[n_free_total]). */
void orc_ising_gamma(const orc_ising *p, const uint8_t *state, float *out);
/* Energy of each chain (ising.rs:151-222), f64 accumulation. */
void orc_ising_energy(const orc_ising *p, uint32_t n_chains, const uint8_t *state,
                      double *out);
/* One sweep of one chain in the reference's op-by-op style (materialised
 * [n,k] f32 intermediates, program.rs:324-393 + spin_gibbs.rs:56-100,
 * 512-637).  Used only as the timed CPU baseline. */
void orc_run_blocks_opbyop(const orc_ising *p, uint64_t key, uint32_t n_chains,
                           uint8_t *state, uint64_t n_iters);

/* ---- categorical (Potts) program: discrete_ebm.rs:456-548,
 *      softmax.rs:60-97,586-710 ------------------------------------------ */
typedef struct orc_potts orc_potts;
/* Edges (eu[e], ev[e]) with W[e][q][q] (W[e][a][b] couples x_u=a, x_v=b),
 * node biases bias[n][q], q in 2..65536; states are uint16_t [C][n_total];
 * global state = free blocks ++ clamped blocks
 * (clamped_off / clamped_nodes may be NULL when n_clamped is 0). */
orc_potts *orc_potts_create(uint32_t n_nodes, uint32_t q, size_t n_edges,
                            const uint32_t *eu, const uint32_t *ev,
                            const float *W, const float *bias, uint32_t n_free,
                            const uint32_t *free_off, const uint32_t *free_nodes,
                            uint32_t n_clamped, const uint32_t *clamped_off,
                            const uint32_t *clamped_nodes, char *err, size_t errlen);
void orc_potts_destroy(orc_potts *p);
/* Superblocks, as orc_ising_set_superblocks. */
int orc_potts_set_superblocks(orc_potts *p, uint32_t n_sb, const uint32_t *off, char *err,
                              size_t errlen);
size_t orc_potts_total(const orc_potts *p);
/* theta[n_total][q] of one chain's state (compute_parameters). */
void orc_potts_theta(const orc_potts *p, const uint16_t *state, float *out);
int64_t orc_potts_pos(const orc_potts *p, uint32_t node);
/* out[c] = -(sum_n b[n][x_n] + sum_e W[e][x_u][x_v]) of chain c's state
 * [C][n_total] (discrete_ebm.rs:551-593 over the bias and edge factors). */
void orc_potts_energy(const orc_potts *p, uint32_t C, const uint16_t *state, double *out);
void orc_potts_run_blocks(const orc_potts *p, uint64_t key, uint32_t n_chains,
                          uint16_t *state, uint64_t n_iters, int n_threads,
                          uint64_t *thr_sites);
/* sample_states of every chain (the same key tree as orc_sample_states):
 * out[n_obs][C][n_total], n_obs = max(n_samples, 1). */
void orc_potts_sample_states(const orc_potts *p, uint64_t key, orc_schedule sched, uint32_t C,
                             uint16_t *state, uint16_t *out, int n_threads);

/* ---- general discrete factors: discrete_ebm.rs:293-593, factor.rs:126-185,
 *      spin_gibbs.rs:512-595, softmax.rs:586-710 -------------------------- */
/* One DiscreteEBMFactor: n_spin spin node groups then n_cat (0..2)
 * categorical node groups of `batch` node ids each (nodes[(g * batch) + b]),
 * weights w[batch][d1][d2]. */
typedef struct {
  uint32_t n_spin, n_cat, batch, d1, d2;
  const uint32_t *nodes;
  const float *w;
  uint32_t square; /* SquareDiscreteEBMFactor: d1 == d2, categorical-head groups merged */
} orc_factor;
typedef struct orc_discrete orc_discrete;
/* node_kind[n] = 0 spin, 1 categorical with q categories (one q for all
 * categorical nodes); free ++ clamped blocks, each of one kind. */
orc_discrete *orc_discrete_create(uint32_t n_nodes, const uint8_t *node_kind, uint32_t q,
                                  uint32_t n_factors, const orc_factor *factors,
                                  uint32_t n_free, const uint32_t *free_off,
                                  const uint32_t *free_nodes, uint32_t n_clamped,
                                  const uint32_t *clamp_off, const uint32_t *clamp_nodes,
                                  char *err, size_t errlen);
void orc_discrete_destroy(orc_discrete *p);
int orc_discrete_set_superblocks(orc_discrete *p, uint32_t n_sb, const uint32_t *off, char *err,
                                 size_t errlen);
size_t orc_discrete_total(const orc_discrete *p);
int64_t orc_discrete_pos(const orc_discrete *p, uint32_t node);
/* gamma (spin position: out[k * max(q,1)]) or theta[0..q) of every free
 * position for one chain's global state */
void orc_discrete_params(const orc_discrete *p, const uint16_t *state, float *out);
void orc_discrete_run_blocks(const orc_discrete *p, uint64_t key, uint32_t n_chains,
                             uint16_t *state, uint64_t n_iters, int n_threads, uint64_t *thr_sites);
void orc_discrete_sample_states(const orc_discrete *p, uint64_t key, orc_schedule sched,
                                uint32_t n_chains, uint16_t *state, uint16_t *out, int n_threads);
void orc_discrete_energy(const orc_discrete *p, uint32_t n_chains, const uint16_t *state,
                         double *out);

/* ---- dense bipartite (RBM-shaped Ising) --------------------------------- */
/* Visible block = nodes 0..V-1, hidden = V..V+H-1; W[v][h] (already rounded
 * to bf16 and widened to f32 by the caller), biases bv[V], bh[H], beta.
 * One half-sweep of block `blk` (0 = visible, 1 = hidden) with the given
 * expanded stream keys key8[c][8] per chain.  gamma in f64 (exact for the
 * bf16 x +-1 products); decisions u <= sigmoid(2*gamma) with gamma rounded
 * to f32.  near[c*n_b+i] (may be NULL) is set to 1 when |2*gamma - logit(u)|
 * < tol. */
void orc_rbm_half_sweep(uint32_t V, uint32_t H, const float *W, const float *bv,
                        const float *bh, float beta, uint32_t n_chains,
                        const uint32_t *key8, int blk, uint8_t *sv, uint8_t *sh,
                        uint8_t *near, double tol, int n_threads);

#ifdef __cplusplus
}
#endif
#endif
