/*
 * orc_ising.c -- oracle restatement of the Ising block Gibbs sweep.
 *
 * TEST INFRASTRUCTURE ONLY (see thrml_oracle.h).
 *
 * Program construction follows
 *   IsingEBM::get_factors             crates/thrml-models/src/ising.rs:105-143
 *     bias factor  W = beta*b  [N,1,1] over all nodes,
 *     edge factor  W = beta*J  [E,1,1] over (U, V);
 *   DiscreteEBMFactor::to_interaction_groups
 *                                      crates/thrml-models/src/discrete_ebm.rs:390-453
 *     edge group head = [u_1..u_E, v_1..v_E], tail = [v_1..v_E, u_1..u_E];
 *   BlockSamplingProgram::new          crates/thrml-samplers/src/program.rs:88-318
 *     per head node, slots in group order and, inside a group, in ascending
 *     head position: for node x the edges with u_e = x (ascending e), then
 *     the edges with v_e = x (ascending e).
 * The conditional follows SpinGibbsConditional
 *   crates/thrml-samplers/src/spin_gibbs.rs:56-100 (sample) and :512-637
 *   gamma = (0 + sum_bias) + sum_k (W_k * active_k) * (2 s_k - 1),
 *   each group summed over its slots first (sequential slot order here),
 *   s' = (u <= sigmoid(2 gamma)).
 * The sweep follows run_blocks / sample_blocks
 *   crates/thrml-samplers/src/sampling.rs:28-106: sweep keys
 *   key.split(n_iters), block keys sweep_key.split(n_blocks).  By default
 *   every free block is its own superblock (ising.rs:348-349), so a block
 *   sees the states written by earlier blocks of the same sweep; with
 *   orc_ising_set_superblocks the blocks of one superblock all read the state
 *   from before it and write after it (sampling.rs:39-60).
 * Build conventions (the reference draws its uniforms from Burn's global RNG
 * and ignores the key, spin_gibbs.rs:61,82-83):
 *   chain c runs with RngKey::split(key, C)[c];
 *   the uniform of block-local site i under block key k is
 *     u = (w >> 8) * 2^-24,  w = word i of ChaCha8Rng::seed_from_u64(k).
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "thrml_oracle.h"

struct orc_ising {
  uint32_t n_nodes;
  size_t n_edges;
  uint32_t n_free, n_clamped;
  size_t n_total;
  uint32_t *blk_off;  /* [n_free+n_clamped+1] position offsets */
  uint32_t *pos_node; /* position -> node */
  int64_t *node_pos;  /* node -> position (or -1) */
  float beta;
  float *bias_raw; /* [N] */
  float *w_raw;    /* [E] */
  uint32_t *eu, *ev;
  int has_bias_group, has_edge_group;
  /* per free position */
  float *bias_w;     /* fl(beta * b) */
  size_t *slot_off;  /* [n_free_total+1] */
  uint32_t *slot_pos;
  float *slot_w;     /* fl(beta * J) */
  size_t n_free_total;
  uint32_t n_sb;
  uint32_t *sb_off; /* [n_sb+1] superblock offsets over the free blocks */
};

static void set_err(char *err, size_t errlen, const char *msg) {
  if (err && errlen) {
    snprintf(err, errlen, "%s", msg);
  }
}

orc_ising *orc_ising_create(uint32_t n_nodes, size_t n_edges, const uint32_t *eu,
                            const uint32_t *ev, const float *bias,
                            const float *weight, float beta, uint32_t n_free,
                            const uint32_t *free_off, const uint32_t *free_nodes,
                            uint32_t n_clamped, const uint32_t *clamp_off,
                            const uint32_t *clamp_nodes, char *err, size_t errlen) {
  orc_ising *p = (orc_ising *)calloc(1, sizeof(orc_ising));
  p->n_nodes = n_nodes;
  p->n_edges = n_edges;
  p->n_free = n_free;
  p->n_clamped = n_clamped;
  p->beta = beta;
  uint32_t nb = n_free + n_clamped;
  p->blk_off = (uint32_t *)malloc((nb + 1) * sizeof(uint32_t));
  p->blk_off[0] = 0;
  for (uint32_t b = 0; b < nb; b++) {
    uint32_t len = b < n_free ? free_off[b + 1] - free_off[b]
                              : clamp_off[b - n_free + 1] - clamp_off[b - n_free];
    if (len == 0) {
      set_err(err, errlen, "Encountered an empty block in BlockSpec");
      orc_ising_destroy(p);
      return NULL;
    }
    p->blk_off[b + 1] = p->blk_off[b] + len;
  }
  p->n_total = p->blk_off[nb];
  p->n_free_total = p->blk_off[n_free];
  p->pos_node = (uint32_t *)malloc((p->n_total + 1) * sizeof(uint32_t));
  p->node_pos = (int64_t *)malloc(((size_t)n_nodes + 1) * sizeof(int64_t));
  for (uint32_t x = 0; x < n_nodes; x++) p->node_pos[x] = -1;
  for (uint32_t b = 0; b < nb; b++) {
    for (uint32_t k = p->blk_off[b]; k < p->blk_off[b + 1]; k++) {
      uint32_t node = b < n_free ? free_nodes[free_off[b] + (k - p->blk_off[b])]
                                 : clamp_nodes[clamp_off[b - n_free] + (k - p->blk_off[b])];
      if (node >= n_nodes) {
        set_err(err, errlen, "Node not found in global location map");
        orc_ising_destroy(p);
        return NULL;
      }
      if (p->node_pos[node] >= 0) {
        set_err(err, errlen, "Node appears twice in blocks");
        orc_ising_destroy(p);
        return NULL;
      }
      p->node_pos[node] = k;
      p->pos_node[k] = node;
    }
  }
  p->bias_raw = (float *)malloc(((size_t)n_nodes + 1) * sizeof(float));
  memcpy(p->bias_raw, bias, (size_t)n_nodes * sizeof(float));
  p->w_raw = (float *)malloc((n_edges + 1) * sizeof(float));
  p->eu = (uint32_t *)malloc((n_edges + 1) * sizeof(uint32_t));
  p->ev = (uint32_t *)malloc((n_edges + 1) * sizeof(uint32_t));
  if (n_edges) {
    memcpy(p->w_raw, weight, n_edges * sizeof(float));
    memcpy(p->eu, eu, n_edges * sizeof(uint32_t));
    memcpy(p->ev, ev, n_edges * sizeof(uint32_t));
  }
  p->has_bias_group = n_nodes > 0;
  p->has_edge_group = n_edges > 0;

  /* slots: count per node (u-role then v-role, ascending e) */
  size_t nf = p->n_free_total;
  p->bias_w = (float *)malloc((nf + 1) * sizeof(float));
  p->slot_off = (size_t *)calloc(nf + 1, sizeof(size_t));
  for (size_t e = 0; e < n_edges; e++) {
    if (eu[e] >= n_nodes || ev[e] >= n_nodes) {
      set_err(err, errlen, "Node not found in global location map");
      orc_ising_destroy(p);
      return NULL;
    }
    int64_t pu = p->node_pos[eu[e]], pv = p->node_pos[ev[e]];
    if (pu >= 0 && (size_t)pu < nf) p->slot_off[pu + 1]++;
    if (pv >= 0 && (size_t)pv < nf) p->slot_off[pv + 1]++;
  }
  for (size_t k = 0; k < nf; k++) p->slot_off[k + 1] += p->slot_off[k];
  size_t ns = p->slot_off[nf];
  p->slot_pos = (uint32_t *)malloc((ns + 1) * sizeof(uint32_t));
  p->slot_w = (float *)malloc((ns + 1) * sizeof(float));
  size_t *fill = (size_t *)malloc((nf + 1) * sizeof(size_t));
  memcpy(fill, p->slot_off, (nf + 1) * sizeof(size_t));
  /* pass 1: u-role slots in ascending e */
  for (size_t e = 0; e < n_edges; e++) {
    int64_t pu = p->node_pos[eu[e]];
    if (pu >= 0 && (size_t)pu < nf) {
      int64_t pt = p->node_pos[ev[e]];
      if (pt < 0) {
        set_err(err, errlen, "Node not found in global location map");
        free(fill);
        orc_ising_destroy(p);
        return NULL;
      }
      p->slot_pos[fill[pu]] = (uint32_t)pt;
      p->slot_w[fill[pu]] = beta * weight[e];
      fill[pu]++;
    }
  }
  /* pass 2: v-role slots in ascending e */
  for (size_t e = 0; e < n_edges; e++) {
    int64_t pv = p->node_pos[ev[e]];
    if (pv >= 0 && (size_t)pv < nf) {
      int64_t pt = p->node_pos[eu[e]];
      if (pt < 0) {
        set_err(err, errlen, "Node not found in global location map");
        free(fill);
        orc_ising_destroy(p);
        return NULL;
      }
      p->slot_pos[fill[pv]] = (uint32_t)pt;
      p->slot_w[fill[pv]] = beta * weight[e];
      fill[pv]++;
    }
  }
  free(fill);
  for (size_t k = 0; k < nf; k++) p->bias_w[k] = beta * bias[p->pos_node[k]];
  p->sb_off = orc_sb_partition(n_free, 0, NULL, &p->n_sb, NULL, 0);
  return p;
}

int orc_ising_set_superblocks(orc_ising *p, uint32_t n_sb, const uint32_t *off, char *err,
                              size_t errlen) {
  uint32_t n = 0;
  uint32_t *r = orc_sb_partition(p->n_free, n_sb, off, &n, err, errlen);
  if (!r) return -1;
  free(p->sb_off);
  p->sb_off = r;
  p->n_sb = n;
  return 0;
}

/* positions of the largest superblock (the staging length of a sweep) */
static size_t ising_max_superblock(const orc_ising *p) {
  size_t m = 0;
  for (uint32_t s = 0; s < p->n_sb; s++) {
    size_t l = p->blk_off[p->sb_off[s + 1]] - p->blk_off[p->sb_off[s]];
    if (l > m) m = l;
  }
  return m;
}

void orc_ising_destroy(orc_ising *p) {
  if (!p) return;
  free(p->blk_off);
  free(p->pos_node);
  free(p->node_pos);
  free(p->bias_raw);
  free(p->w_raw);
  free(p->eu);
  free(p->ev);
  free(p->bias_w);
  free(p->slot_off);
  free(p->slot_pos);
  free(p->slot_w);
  free(p->sb_off);
  free(p);
}

size_t orc_ising_total(const orc_ising *p) { return p->n_total; }
int64_t orc_ising_pos(const orc_ising *p, uint32_t node) {
  return node < p->n_nodes ? p->node_pos[node] : -1;
}

/* gamma of free position k for one chain's global state st */
static float gamma_at(const orc_ising *p, size_t k, const uint8_t *st) {
  float g = 0.0f;
  if (p->has_bias_group) g = g + p->bias_w[k];
  if (p->has_edge_group) {
    size_t a = p->slot_off[k], b = p->slot_off[k + 1];
    float acc = 0.0f;
    for (size_t s = a; s < b; s++) {
      float sp = st[p->slot_pos[s]] ? 1.0f : -1.0f;
      float t = p->slot_w[s] * sp;
      acc = (s == a) ? t : acc + t;
    }
    g = g + acc;
  }
  return g;
}

static int near_threshold(float gamma, float u) {
  if (u <= 0.0f) return 0;
  double lu = log((double)u / (1.0 - (double)u));
  return fabs(2.0 * (double)gamma - lu) < 1e-5;
}

/* one block update of one chain with the expanded block key k8: the new
 * states go to tmp[0..n_b) and st is only read */
static uint64_t update_block(const orc_ising *p, uint32_t b, const uint32_t k8[8],
                             const uint8_t *st, uint8_t *tmp) {
  uint32_t off = p->blk_off[b], n = p->blk_off[b + 1] - off;
  uint32_t blk[16];
  uint64_t near = 0;
  for (uint32_t i = 0; i < n; i++) {
    if ((i & 15u) == 0) orc_chacha_block(k8, i >> 4, 0, 8, blk);
    float g = gamma_at(p, off + i, st);
    float prob = orc_sigmoid(g * 2.0f);
    float u = (float)(blk[i & 15u] >> 8) * 0x1p-24f;
    tmp[i] = (uint8_t)(u <= prob);
    near += (uint64_t)near_threshold(g, u);
  }
  return near;
}

/* One sweep of one chain with block keys bk[n_free]: the superblocks in
 * order; the blocks of a superblock all read st as it was before the
 * superblock and their new states replace the old ones after it
 * (sampling.rs:39-60).  tmp holds ising_max_superblock(p) bytes. */
static uint64_t sweep_chain(const orc_ising *p, const uint64_t *bk, uint8_t *st, uint8_t *tmp) {
  uint64_t near = 0;
  for (uint32_t s = 0; s < p->n_sb; s++) {
    const uint32_t first = p->sb_off[s], end = p->sb_off[s + 1];
    if (first == end) continue;
    const uint32_t base = p->blk_off[first];
    for (uint32_t b = first; b < end; b++) {
      uint32_t k8[8];
      orc_seed_from_u64(bk[b], k8);
      near += update_block(p, b, k8, st, tmp + (p->blk_off[b] - base));
    }
    memcpy(st + base, tmp, p->blk_off[end] - base);
  }
  return near;
}

static void chain_keys(uint64_t key, uint32_t C, uint64_t *out) {
  orc_rng_split(key, C, out);
}

static uint64_t run_chain(const orc_ising *p, uint64_t ckey, uint8_t *st,
                          uint64_t n_iters, uint8_t *tmp) {
  if (n_iters == 0) return 0;
  uint64_t *sk = (uint64_t *)malloc(n_iters * sizeof(uint64_t));
  uint64_t *bk = (uint64_t *)malloc((p->n_free + 1) * sizeof(uint64_t));
  orc_rng_split(ckey, n_iters, sk);
  uint64_t near = 0;
  for (uint64_t s = 0; s < n_iters; s++) {
    orc_rng_split(sk[s], p->n_free, bk);
    near += sweep_chain(p, bk, st, tmp);
  }
  free(sk);
  free(bk);
  return near;
}

void orc_run_blocks(const orc_ising *p, uint64_t key, uint32_t C, uint8_t *state,
                    uint64_t n_iters, int n_threads, uint64_t *thr_sites) {
  uint64_t *ck = (uint64_t *)malloc(((size_t)C + 1) * sizeof(uint64_t));
  chain_keys(key, C, ck);
  uint64_t near = 0;
  const size_t maxb = ising_max_superblock(p);
#pragma omp parallel for schedule(dynamic, 1) num_threads(n_threads > 0 ? n_threads : 1) reduction(+ : near)
  for (int64_t c = 0; c < (int64_t)C; c++) {
    uint8_t *tmp = (uint8_t *)malloc(maxb + 1);
    near += run_chain(p, ck[c], state + (size_t)c * p->n_total, n_iters, tmp);
    free(tmp);
  }
  free(ck);
  if (thr_sites) *thr_sites = near;
}

void orc_run_blocks_subset(const orc_ising *p, uint64_t key, uint32_t C_total,
                           const uint32_t *chains, uint32_t n_sel, uint8_t *state,
                           uint64_t n_iters, int n_threads) {
  uint64_t *ck = (uint64_t *)malloc(((size_t)C_total + 1) * sizeof(uint64_t));
  chain_keys(key, C_total, ck);
  const size_t maxb = ising_max_superblock(p);
#pragma omp parallel for schedule(dynamic, 1) num_threads(n_threads > 0 ? n_threads : 1)
  for (int64_t k = 0; k < (int64_t)n_sel; k++) {
    uint8_t *tmp = (uint8_t *)malloc(maxb + 1);
    run_chain(p, ck[chains[k]], state + (size_t)k * p->n_total, n_iters, tmp);
    free(tmp);
  }
  free(ck);
}

void orc_ising_gamma(const orc_ising *p, const uint8_t *state, float *out) {
  for (size_t k = 0; k < p->n_free_total; k++) out[k] = gamma_at(p, k, state);
}

void orc_hinton_init(const orc_ising *p, uint64_t key, uint32_t C, uint8_t *state) {
  /* ising.rs:602-673: p = sigmoid(b * beta) per block node, samples
   * (u <= p) for a [batch, block_len] uniform tensor.  Build convention:
   * block b uses key.split(n_blocks)[b]; entry (c, i) takes word c*n_b + i. */
  uint64_t *bk = (uint64_t *)malloc((p->n_free + 1) * sizeof(uint64_t));
  orc_rng_split(key, p->n_free, bk);
  for (uint32_t b = 0; b < p->n_free; b++) {
    uint32_t k8[8];
    orc_seed_from_u64(bk[b], k8);
    uint32_t off = p->blk_off[b], n = p->blk_off[b + 1] - off;
    uint32_t blk[16];
    uint64_t cur = (uint64_t)-1;
    for (uint32_t c = 0; c < C; c++) {
      for (uint32_t i = 0; i < n; i++) {
        uint64_t w = (uint64_t)c * n + i;
        if ((w >> 4) != cur) {
          cur = w >> 4;
          orc_chacha_block(k8, cur, 0, 8, blk);
        }
        float prob = orc_sigmoid(p->bias_raw[p->pos_node[off + i]] * p->beta);
        float u = (float)(blk[w & 15] >> 8) * 0x1p-24f;
        state[(size_t)c * p->n_total + off + i] = (uint8_t)(u <= prob);
      }
    }
  }
  free(bk);
}

/* hinton uses sigmoid(b*beta) without the factor 2: keep the call above
 * literal; orc_sigmoid clamps its argument itself. */

static void observe(const orc_ising *p, const uint8_t *st, const int64_t *npos,
                    size_t n1, const int64_t *ppos, size_t n2, int64_t *ns,
                    int64_t *es) {
  for (size_t k = 0; k < n1; k++) ns[k] += st[npos[k]] ? 1 : -1;
  for (size_t k = 0; k < n2; k++) {
    int a = st[ppos[2 * k]] ? 1 : -1;
    int b = st[ppos[2 * k + 1]] ? 1 : -1;
    es[k] += a * b;
  }
  (void)p;
}

void orc_estimate_moments(const orc_ising *p, uint64_t key, orc_schedule sched,
                          uint32_t C, uint8_t *state, const uint32_t *nodes,
                          size_t n1, const uint32_t *pairs, size_t n2,
                          int64_t *node_sums, int64_t *edge_sums, int n_threads,
                          uint64_t *thr_sites) {
  int64_t *npos = (int64_t *)malloc((n1 + 1) * sizeof(int64_t));
  int64_t *ppos = (int64_t *)malloc((2 * n2 + 1) * sizeof(int64_t));
  for (size_t k = 0; k < n1; k++) npos[k] = p->node_pos[nodes[k]];
  for (size_t k = 0; k < 2 * n2; k++) ppos[k] = p->node_pos[pairs[k]];
  memset(node_sums, 0, n1 * sizeof(int64_t));
  memset(edge_sums, 0, n2 * sizeof(int64_t));
  uint64_t *ck = (uint64_t *)malloc(((size_t)C + 1) * sizeof(uint64_t));
  chain_keys(key, C, ck);
  const size_t maxb = ising_max_superblock(p);
  uint64_t near = 0;
#pragma omp parallel num_threads(n_threads > 0 ? n_threads : 1) reduction(+ : near)
  {
    int64_t *ns = (int64_t *)calloc(n1 + 1, sizeof(int64_t));
    int64_t *es = (int64_t *)calloc(n2 + 1, sizeof(int64_t));
    uint8_t *tmp = (uint8_t *)malloc(maxb + 1);
#pragma omp for schedule(dynamic, 1)
    for (int64_t c = 0; c < (int64_t)C; c++) {
      uint8_t *st = state + (size_t)c * p->n_total;
      uint64_t wk_sk[2];
      orc_rng_split(ck[c], 2, wk_sk); /* sampling.rs:189 */
      near += run_chain(p, wk_sk[0], st, sched.n_warmup, tmp);
      observe(p, st, npos, n1, ppos, n2, ns, es); /* :200 */
      if (sched.n_samples > 1) {
        uint64_t m = sched.n_samples - 1;
        uint64_t *keys = (uint64_t *)malloc(m * sizeof(uint64_t));
        orc_rng_split(wk_sk[1], m, keys); /* :222 */
        for (uint64_t i = 0; i < m; i++) {
          near += run_chain(p, keys[i], st, sched.steps_per_sample, tmp);
          observe(p, st, npos, n1, ppos, n2, ns, es);
        }
        free(keys);
      }
    }
#pragma omp critical
    {
      for (size_t k = 0; k < n1; k++) node_sums[k] += ns[k];
      for (size_t k = 0; k < n2; k++) edge_sums[k] += es[k];
    }
    free(ns);
    free(es);
    free(tmp);
  }
  free(ck);
  free(npos);
  free(ppos);
  if (thr_sites) *thr_sites = near;
}

/* sample_with_observation with a StateObserver over every node
 * (sampling.rs:128-156,178-320, state_observer.rs:22-48): the same key tree
 * as orc_estimate_moments, the whole global state copied out after the
 * warmup and after each later sample, out[n_obs][C][n_total]. */
void orc_sample_states(const orc_ising *p, uint64_t key, orc_schedule sched,
                       uint32_t C, uint8_t *state, uint8_t *out, int n_threads) {
  const uint64_t n_obs = sched.n_samples > 1 ? sched.n_samples : 1;
  uint64_t *ck = (uint64_t *)malloc(((size_t)C + 1) * sizeof(uint64_t));
  chain_keys(key, C, ck);
  const size_t maxb = ising_max_superblock(p);
#pragma omp parallel num_threads(n_threads > 0 ? n_threads : 1)
  {
    uint8_t *tmp = (uint8_t *)malloc(maxb + 1);
#pragma omp for schedule(dynamic, 1)
    for (int64_t c = 0; c < (int64_t)C; c++) {
      uint8_t *st = state + (size_t)c * p->n_total;
      uint64_t wk_sk[2];
      orc_rng_split(ck[c], 2, wk_sk);
      run_chain(p, wk_sk[0], st, sched.n_warmup, tmp);
      memcpy(out + (size_t)c * p->n_total, st, p->n_total);
      if (n_obs > 1) {
        uint64_t m = n_obs - 1;
        uint64_t *keys = (uint64_t *)malloc(m * sizeof(uint64_t));
        orc_rng_split(wk_sk[1], m, keys);
        for (uint64_t i = 0; i < m; i++) {
          run_chain(p, keys[i], st, sched.steps_per_sample, tmp);
          memcpy(out + ((size_t)(i + 1) * C + c) * p->n_total, st, p->n_total);
        }
        free(keys);
      }
    }
    free(tmp);
  }
  free(ck);
}

void orc_ising_energy(const orc_ising *p, uint32_t C, const uint8_t *state,
                      double *out) {
  for (uint32_t c = 0; c < C; c++) {
    const uint8_t *st = state + (size_t)c * p->n_total;
    double eb = 0.0, ee = 0.0;
    for (uint32_t x = 0; x < p->n_nodes; x++) {
      if (p->node_pos[x] < 0) continue;
      eb += (double)p->bias_raw[x] * (st[p->node_pos[x]] ? 1.0 : -1.0);
    }
    for (size_t e = 0; e < p->n_edges; e++) {
      int64_t a = p->node_pos[p->eu[e]], b = p->node_pos[p->ev[e]];
      if (a < 0 || b < 0) continue;
      double sa = st[a] ? 1.0 : -1.0, sb = st[b] ? 1.0 : -1.0;
      ee += (double)p->w_raw[e] * sa * sb;
    }
    out[c] = -(double)p->beta * (eb + ee);
  }
}

/* ---- op-by-op baseline (reference execution style) ---------------------- */
void orc_run_blocks_opbyop(const orc_ising *p, uint64_t key, uint32_t C,
                           uint8_t *state, uint64_t n_iters) {
  /* Mirrors the Burn op sequence of program.rs:333-366 and
   * spin_gibbs.rs:56-100,512-637 for one chain at a time: global state as
   * f32, per block the padded [n, k] gather, 2s-1, W*active, *spin_prod,
   * sum_dim, gamma add, uniform tensor, *2, sigmoid, lower_equal, float. */
  uint64_t *ck = (uint64_t *)malloc(((size_t)C + 1) * sizeof(uint64_t));
  chain_keys(key, C, ck);
  size_t nt = p->n_total;
  float *glob = (float *)malloc((nt + 1) * sizeof(float));
  uint8_t *pre = (uint8_t *)malloc(nt + 1); /* the state before a superblock of 2+ blocks */
  for (uint32_t c = 0; c < C; c++) {
    uint8_t *st = state + (size_t)c * nt;
    uint64_t *sk = (uint64_t *)malloc((n_iters + 1) * sizeof(uint64_t));
    orc_rng_split(ck[c], n_iters, sk);
    for (uint64_t s = 0; s < n_iters; s++) {
      uint64_t bk[64];
      uint64_t *bkp = p->n_free <= 64 ? bk : (uint64_t *)malloc(p->n_free * sizeof(uint64_t));
      orc_rng_split(sk[s], p->n_free, bkp);
      uint32_t sb = 0;
      const uint8_t *src = st;
      for (uint32_t b = 0; b < p->n_free; b++) {
        while (p->sb_off[sb + 1] <= b) sb++;
        if (b == p->sb_off[sb]) {
          /* state_free is updated only after a superblock (sampling.rs:39-60) */
          src = st;
          if (p->sb_off[sb + 1] - b > 1) {
            memcpy(pre, st, nt);
            src = pre;
          }
        }
        uint32_t off = p->blk_off[b], n = p->blk_off[b + 1] - off;
        /* block_state_to_global: Tensor::cat of all blocks (program.rs:333) */
        for (size_t k = 0; k < nt; k++) glob[k] = (float)src[k];
        size_t kmax = 0;
        for (uint32_t i = 0; i < n; i++) {
          size_t d = p->slot_off[off + i + 1] - p->slot_off[off + i];
          if (d > kmax) kmax = d;
        }
        size_t nk = (size_t)n * (kmax ? kmax : 1);
        float *gath = (float *)calloc(nk, sizeof(float));
        float *wsl = (float *)calloc(nk, sizeof(float));
        float *act = (float *)calloc(nk, sizeof(float));
        float *gam = (float *)calloc(n, sizeof(float));
        float *uni = (float *)malloc(n * sizeof(float));
        /* bias group: [n,1] W*1*1 summed */
        for (uint32_t i = 0; i < n; i++) gam[i] = gam[i] + p->bias_w[off + i];
        if (kmax) {
          for (uint32_t i = 0; i < n; i++) {
            size_t a = p->slot_off[off + i], d = p->slot_off[off + i + 1] - a;
            for (size_t j = 0; j < kmax; j++) {
              size_t q = (size_t)i * kmax + j;
              if (j < d) {
                gath[q] = glob[p->slot_pos[a + j]];
                wsl[q] = p->slot_w[a + j];
                act[q] = 1.0f;
              } else {
                gath[q] = glob[0];
                wsl[q] = p->slot_w[0];
                act[q] = 0.0f;
              }
            }
          }
          for (size_t q = 0; q < nk; q++) gath[q] = gath[q] * 2.0f - 1.0f;
          for (size_t q = 0; q < nk; q++) wsl[q] = wsl[q] * act[q];
          for (size_t q = 0; q < nk; q++) wsl[q] = wsl[q] * gath[q];
          for (uint32_t i = 0; i < n; i++) {
            float acc = 0.0f;
            for (size_t j = 0; j < kmax; j++) acc = j ? acc + wsl[(size_t)i * kmax + j] : wsl[(size_t)i * kmax + j];
            gam[i] = gam[i] + acc;
          }
        }
        uint32_t k8[8], blk[16];
        orc_seed_from_u64(bkp[b], k8);
        for (uint32_t i = 0; i < n; i++) {
          if ((i & 15u) == 0) orc_chacha_block(k8, i >> 4, 0, 8, blk);
          uni[i] = (float)(blk[i & 15u] >> 8) * 0x1p-24f;
        }
        for (uint32_t i = 0; i < n; i++) gam[i] = gam[i] * 2.0f;
        for (uint32_t i = 0; i < n; i++) gam[i] = orc_sigmoid(gam[i]);
        for (uint32_t i = 0; i < n; i++) st[off + i] = (uint8_t)(uni[i] <= gam[i]);
        free(gath);
        free(wsl);
        free(act);
        free(gam);
        free(uni);
      }
      if (bkp != bk) free(bkp);
    }
    free(sk);
  }
  free(glob);
  free(pre);
  free(ck);
}
