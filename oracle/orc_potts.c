/*
 * orc_potts.c -- oracle restatement of the categorical (Potts) Gibbs sweep.
 *
 * TEST INFRASTRUCTURE ONLY (see thrml_oracle.h).
 *
 * Model: a bias factor CategoricalEBMFactor([all nodes], b[N, q]) followed by
 * an edge factor CategoricalEBMFactor([U, V], W[E, q, q]).
 * DiscreteEBMFactor::to_interaction_groups
 *   (crates/thrml-models/src/discrete_ebm.rs:456-507) yields, in order,
 *   the bias group, the group with head U / tail V and weights W, and the
 *   group with head V / tail U and weights W.swap_dims(1, 2) (:518-548).
 * CategoricalGibbsConditional::compute_parameters
 *   (crates/thrml-samplers/src/softmax.rs:586-710):
 *   theta[c] = ((0 + b[x][c]) + sum_{e: u_e=x} W[e][c][x_v])
 *                             + sum_{e: v_e=x} W[e][x_u][c],
 *   each group summed over its slots (ascending e) before it is added.
 * categorical_sample (softmax.rs:60-97): argmax_c(theta_c - log(-log u_c)),
 *   first maximum on ties (crates/thrml-kernels/src/gumbel_argmax/kernel.rs:81-83).
 * Build convention for the uniforms: site i, category c of a block with key k
 *   takes word i*q + c of ChaCha8Rng::seed_from_u64(k); u = ((w>>8)|1) 2^-24.
 * States hold one uint16_t per (chain, position): q is 2..65536 (the
 *   reference takes any q).
 * Blocks: the global state is the free blocks then the clamped blocks
 *   (crates/thrml-core/src/blockspec.rs:15-67); only free blocks are updated,
 *   clamped positions are read as tails (state_clamp, sampling.rs:81-106).
 *   Superblocks (orc_potts_set_superblocks): the blocks of one read the state
 *   from before it and write after it (sampling.rs:39-60).
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "thrml_oracle.h"

struct orc_potts {
  uint32_t n_nodes, q, n_free, n_clamped;
  size_t n_edges, n_total;
  uint32_t *blk_off, *pos_node;
  int64_t *node_pos;
  float *bias; /* [N][q] */
  float *W;    /* [E][q][q] */
  /* per position: u-role slots then v-role slots */
  size_t *uoff, *voff;
  uint32_t *u_tail, *u_edge, *v_tail, *v_edge;
  uint32_t *epu, *epv; /* endpoint positions of every edge, edge order */
  int has_u_group, has_v_group;
  uint32_t n_sb;
  uint32_t *sb_off; /* [n_sb+1] superblock offsets over the free blocks */
};

orc_potts *orc_potts_create(uint32_t n_nodes, uint32_t q, size_t n_edges,
                            const uint32_t *eu, const uint32_t *ev, const float *W,
                            const float *bias, uint32_t n_free,
                            const uint32_t *free_off, const uint32_t *free_nodes,
                            uint32_t n_clamped, const uint32_t *clamped_off,
                            const uint32_t *clamped_nodes, char *err, size_t errlen) {
  if (q < 2 || q > ORC_POTTS_MAX_Q) {
    if (err) snprintf(err, errlen, "q must lie in 2..65536");
    return NULL;
  }
  orc_potts *p = (orc_potts *)calloc(1, sizeof(orc_potts));
  p->n_nodes = n_nodes;
  p->q = q;
  p->n_free = n_free;
  p->n_clamped = n_clamped;
  p->n_edges = n_edges;
  const uint32_t nb = n_free + n_clamped;
  p->blk_off = (uint32_t *)malloc((nb + 1) * sizeof(uint32_t));
  p->blk_off[0] = 0;
  for (uint32_t b = 0; b < nb; b++) {
    const uint32_t len = b < n_free ? free_off[b + 1] - free_off[b]
                                    : clamped_off[b - n_free + 1] - clamped_off[b - n_free];
    if (len == 0) {
      if (err) snprintf(err, errlen, "Encountered an empty block in BlockSpec");
      orc_potts_destroy(p);
      return NULL;
    }
    p->blk_off[b + 1] = p->blk_off[b] + len;
  }
  p->n_total = p->blk_off[nb];
  p->pos_node = (uint32_t *)malloc((p->n_total + 1) * sizeof(uint32_t));
  p->node_pos = (int64_t *)malloc(((size_t)n_nodes + 1) * sizeof(int64_t));
  for (uint32_t x = 0; x < n_nodes; x++) p->node_pos[x] = -1;
  const size_t n_free_total = p->blk_off[n_free];
  for (size_t k = 0; k < p->n_total; k++) {
    uint32_t node = k < n_free_total ? free_nodes[k] : clamped_nodes[k - n_free_total];
    if (node >= n_nodes || p->node_pos[node] >= 0) {
      if (err) snprintf(err, errlen, node >= n_nodes ? "Node not found in global location map" : "Node appears twice in blocks");
      orc_potts_destroy(p);
      return NULL;
    }
    p->node_pos[node] = (int64_t)k;
    p->pos_node[k] = node;
  }
  p->bias = (float *)malloc(((size_t)n_nodes * q + 1) * sizeof(float));
  memcpy(p->bias, bias, (size_t)n_nodes * q * sizeof(float));
  p->W = (float *)malloc((n_edges * q * q + 1) * sizeof(float));
  memcpy(p->W, W, n_edges * q * q * sizeof(float));
  size_t nt = p->n_total;
  p->uoff = (size_t *)calloc(nt + 1, sizeof(size_t));
  p->voff = (size_t *)calloc(nt + 1, sizeof(size_t));
  for (size_t e = 0; e < n_edges; e++) {
    if (eu[e] >= n_nodes || ev[e] >= n_nodes || p->node_pos[eu[e]] < 0 || p->node_pos[ev[e]] < 0) {
      if (err) snprintf(err, errlen, "Node not found in global location map");
      orc_potts_destroy(p);
      return NULL;
    }
    p->uoff[p->node_pos[eu[e]] + 1]++;
    p->voff[p->node_pos[ev[e]] + 1]++;
  }
  for (size_t k = 0; k < nt; k++) {
    p->uoff[k + 1] += p->uoff[k];
    p->voff[k + 1] += p->voff[k];
  }
  p->epu = (uint32_t *)malloc((n_edges + 1) * sizeof(uint32_t));
  p->epv = (uint32_t *)malloc((n_edges + 1) * sizeof(uint32_t));
  for (size_t e = 0; e < n_edges; e++) {
    p->epu[e] = (uint32_t)p->node_pos[eu[e]];
    p->epv[e] = (uint32_t)p->node_pos[ev[e]];
  }
  p->u_tail = (uint32_t *)malloc((n_edges + 1) * sizeof(uint32_t));
  p->u_edge = (uint32_t *)malloc((n_edges + 1) * sizeof(uint32_t));
  p->v_tail = (uint32_t *)malloc((n_edges + 1) * sizeof(uint32_t));
  p->v_edge = (uint32_t *)malloc((n_edges + 1) * sizeof(uint32_t));
  size_t *fu = (size_t *)malloc((nt + 1) * sizeof(size_t));
  size_t *fv = (size_t *)malloc((nt + 1) * sizeof(size_t));
  memcpy(fu, p->uoff, (nt + 1) * sizeof(size_t));
  memcpy(fv, p->voff, (nt + 1) * sizeof(size_t));
  for (size_t e = 0; e < n_edges; e++) {
    size_t pu = (size_t)p->node_pos[eu[e]], pv = (size_t)p->node_pos[ev[e]];
    p->u_tail[fu[pu]] = (uint32_t)pv;
    p->u_edge[fu[pu]++] = (uint32_t)e;
    p->v_tail[fv[pv]] = (uint32_t)pu;
    p->v_edge[fv[pv]++] = (uint32_t)e;
  }
  free(fu);
  free(fv);
  p->has_u_group = n_edges > 0;
  p->has_v_group = n_edges > 0;
  p->sb_off = orc_sb_partition(n_free, 0, NULL, &p->n_sb, NULL, 0);
  return p;
}

int orc_potts_set_superblocks(orc_potts *p, uint32_t n_sb, const uint32_t *off, char *err,
                              size_t errlen) {
  uint32_t n = 0;
  uint32_t *r = orc_sb_partition(p->n_free, n_sb, off, &n, err, errlen);
  if (!r) return -1;
  free(p->sb_off);
  p->sb_off = r;
  p->n_sb = n;
  return 0;
}

void orc_potts_destroy(orc_potts *p) {
  if (!p) return;
  free(p->blk_off);
  free(p->pos_node);
  free(p->node_pos);
  free(p->bias);
  free(p->W);
  free(p->uoff);
  free(p->voff);
  free(p->u_tail);
  free(p->u_edge);
  free(p->v_tail);
  free(p->v_edge);
  free(p->epu);
  free(p->epv);
  free(p->sb_off);
  free(p);
}

size_t orc_potts_total(const orc_potts *p) { return p->n_total; }

/* su, sv: q floats of scratch each */
static void potts_theta(const orc_potts *p, size_t k, const uint16_t *st, float *theta, float *su,
                        float *sv) {
  const uint32_t q = p->q;
  uint32_t x = p->pos_node[k];
  for (uint32_t c = 0; c < q; c++) theta[c] = 0.0f + p->bias[(size_t)x * q + c];
  if (p->has_u_group) {
    for (uint32_t c = 0; c < q; c++) su[c] = 0.0f;
    for (size_t s = p->uoff[k]; s < p->uoff[k + 1]; s++) {
      uint32_t xt = st[p->u_tail[s]];
      const float *We = p->W + (size_t)p->u_edge[s] * q * q;
      for (uint32_t c = 0; c < q; c++) {
        float t = We[(size_t)c * q + xt];
        su[c] = (s == p->uoff[k]) ? t : su[c] + t;
      }
    }
    for (uint32_t c = 0; c < q; c++) theta[c] = theta[c] + su[c];
  }
  if (p->has_v_group) {
    for (uint32_t c = 0; c < q; c++) sv[c] = 0.0f;
    for (size_t s = p->voff[k]; s < p->voff[k + 1]; s++) {
      uint32_t xt = st[p->v_tail[s]];
      const float *We = p->W + (size_t)p->v_edge[s] * q * q;
      for (uint32_t c = 0; c < q; c++) {
        float t = We[(size_t)xt * q + c];
        sv[c] = (s == p->voff[k]) ? t : sv[c] + t;
      }
    }
    for (uint32_t c = 0; c < q; c++) theta[c] = theta[c] + sv[c];
  }
}

void orc_potts_theta(const orc_potts *p, const uint16_t *state, float *out) {
  float *su = (float *)malloc(2 * (size_t)p->q * sizeof(float));
  for (size_t k = 0; k < p->n_total; k++) potts_theta(p, k, state, out + k * p->q, su, su + p->q);
  free(su);
}

int64_t orc_potts_pos(const orc_potts *p, uint32_t node) { return p->node_pos[node]; }

/* one block of one chain: the new categories go to tmp[0..n_b), st is only read */
static uint64_t potts_block(const orc_potts *p, uint32_t b, const uint32_t k8[8],
                            const uint16_t *st, uint16_t *tmp) {
  const uint32_t q = p->q;
  uint32_t off = p->blk_off[b], n = p->blk_off[b + 1] - off;
  float *theta = (float *)malloc(3 * (size_t)q * sizeof(float));
  uint32_t blk[16];
  uint64_t cur = (uint64_t)-1, near = 0;
  for (uint32_t i = 0; i < n; i++) {
    size_t k = off + i;
    potts_theta(p, k, st, theta, theta + q, theta + 2 * (size_t)q);
    float best = 0.0f, second = -INFINITY;
    uint32_t arg = 0;
    for (uint32_t c = 0; c < q; c++) {
      uint64_t w = (uint64_t)i * q + c;
      if ((w >> 4) != cur) {
        cur = w >> 4;
        orc_chacha_block(k8, cur, 0, 8, blk);
      }
      float v = theta[c] + orc_gumbel(blk[w & 15]);
      if (c == 0) {
        best = v;
      } else if (v > best) {
        second = best;
        best = v;
        arg = c;
      } else if (v > second) {
        second = v;
      }
    }
    tmp[i] = (uint16_t)arg;
    if (q > 1 && (double)best - (double)second < 1e-5) near++;
  }
  free(theta);
  return near;
}

/* positions of the largest superblock (the staging length of a sweep) */
static size_t potts_max_block(const orc_potts *p) {
  size_t m = 0;
  for (uint32_t s = 0; s < p->n_sb; s++) {
    size_t l = p->blk_off[p->sb_off[s + 1]] - p->blk_off[p->sb_off[s]];
    if (l > m) m = l;
  }
  return m;
}

/* run_blocks of one chain (sampling.rs:81-106): sweep s takes
 * ckey.split(n_iters)[s], block b of it sweep_key.split(n_free)[b]. */
static uint64_t potts_chain(const orc_potts *p, uint64_t ckey, uint16_t *st, uint64_t n_iters,
                            uint16_t *tmp) {
  if (n_iters == 0) return 0;
  uint64_t near = 0;
  uint64_t *sk = (uint64_t *)malloc(n_iters * sizeof(uint64_t));
  uint64_t *bk = (uint64_t *)malloc((p->n_free + 1) * sizeof(uint64_t));
  orc_rng_split(ckey, n_iters, sk);
  for (uint64_t s = 0; s < n_iters; s++) {
    orc_rng_split(sk[s], p->n_free, bk);
    /* superblocks in order; the new categories of a superblock replace the
     * old ones after its last block (sampling.rs:39-60) */
    for (uint32_t g = 0; g < p->n_sb; g++) {
      const uint32_t first = p->sb_off[g], end = p->sb_off[g + 1];
      if (first == end) continue;
      const uint32_t base = p->blk_off[first];
      for (uint32_t b = first; b < end; b++) {
        uint32_t k8[8];
        orc_seed_from_u64(bk[b], k8);
        near += potts_block(p, b, k8, st, tmp + (p->blk_off[b] - base));
      }
      memcpy(st + base, tmp, (p->blk_off[end] - base) * sizeof(uint16_t));
    }
  }
  free(sk);
  free(bk);
  return near;
}

void orc_potts_run_blocks(const orc_potts *p, uint64_t key, uint32_t C,
                          uint16_t *state, uint64_t n_iters, int n_threads,
                          uint64_t *thr_sites) {
  uint64_t *ck = (uint64_t *)malloc(((size_t)C + 1) * sizeof(uint64_t));
  orc_rng_split(key, C, ck);
  const size_t maxb = potts_max_block(p);
  uint64_t near = 0;
#pragma omp parallel for schedule(dynamic, 1) num_threads(n_threads > 0 ? n_threads : 1) reduction(+ : near)
  for (int64_t c = 0; c < (int64_t)C; c++) {
    uint16_t *tmp = (uint16_t *)malloc((maxb + 1) * sizeof(uint16_t));
    near += potts_chain(p, ck[c], state + (size_t)c * p->n_total, n_iters, tmp);
    free(tmp);
  }
  free(ck);
  if (thr_sites) *thr_sites = near;
}

/* sample_states with a StateObserver over every node (sampling.rs:128-156,
 * 178-320): per chain (wk, sk) = key.split_two(); n_warmup sweeps keyed by
 * wk, observation; then for i < n_samples - 1, steps_per_sample sweeps keyed
 * by sk.split(n_samples - 1)[i], observation.  out[n_obs][C][n_total]. */
void orc_potts_sample_states(const orc_potts *p, uint64_t key, orc_schedule sched, uint32_t C,
                             uint16_t *state, uint16_t *out, int n_threads) {
  const uint64_t n_obs = sched.n_samples > 1 ? sched.n_samples : 1;
  uint64_t *ck = (uint64_t *)malloc(((size_t)C + 1) * sizeof(uint64_t));
  orc_rng_split(key, C, ck);
  const size_t maxb = potts_max_block(p);
#pragma omp parallel for schedule(dynamic, 1) num_threads(n_threads > 0 ? n_threads : 1)
  for (int64_t c = 0; c < (int64_t)C; c++) {
    uint16_t *st = state + (size_t)c * p->n_total;
    uint16_t *tmp = (uint16_t *)malloc((maxb + 1) * sizeof(uint16_t));
    uint64_t wk_sk[2];
    orc_rng_split(ck[c], 2, wk_sk);
    potts_chain(p, wk_sk[0], st, sched.n_warmup, tmp);
    memcpy(out + (size_t)c * p->n_total, st, p->n_total * sizeof(uint16_t));
    if (n_obs > 1) {
      const uint64_t m = n_obs - 1;
      uint64_t *keys = (uint64_t *)malloc(m * sizeof(uint64_t));
      orc_rng_split(wk_sk[1], m, keys);
      for (uint64_t i = 0; i < m; i++) {
        potts_chain(p, keys[i], st, sched.steps_per_sample, tmp);
        memcpy(out + ((size_t)(i + 1) * C + c) * p->n_total, st, p->n_total * sizeof(uint16_t));
      }
      free(keys);
    }
    free(tmp);
  }
  free(ck);
}

/* Energy of each chain: the bias factor's and the edge factor's
 * DiscreteEBMFactor::factor_energy (crates/thrml-models/src/discrete_ebm.rs:551-593),
 * -sum(batch_gather(W, categories)), added: E = -(sum_n b[n][x_n] +
 * sum_e W[e][x_u][x_v]), in double, nodes then edges in index order. */
void orc_potts_energy(const orc_potts *p, uint32_t C, const uint16_t *state, double *out) {
  const uint32_t q = p->q;
  for (uint32_t c = 0; c < C; c++) {
    const uint16_t *st = state + (size_t)c * p->n_total;
    double eb = 0.0, ee = 0.0;
    for (uint32_t x = 0; x < p->n_nodes; x++) {
      if (p->node_pos[x] < 0) continue;
      eb += (double)p->bias[(size_t)x * q + st[p->node_pos[x]]];
    }
    for (size_t e = 0; e < p->n_edges; e++)
      ee += (double)p->W[(e * q + st[p->epu[e]]) * q + st[p->epv[e]]];
    out[c] = -(eb + ee);
  }
}
