/*
 * orc_discrete.c -- oracle restatement of block Gibbs sampling over general
 * discrete factors (spin and categorical nodes).
 *
 * TEST INFRASTRUCTURE ONLY (see thrml_oracle.h).
 *
 * Model: DiscreteEBMFactor (crates/thrml-models/src/discrete_ebm.rs:293-359):
 * n_spin spin node groups and n_cat (0..2) categorical node groups of `batch`
 * nodes each, weights [batch][d1][d2].
 * Interaction groups (to_interaction_groups, discrete_ebm.rs:371-490), per
 * factor in order (FactorSamplingProgram::new, crates/thrml-models/src/factor.rs:
 * 153-185):
 *   - with n_spin > 0, one group whose head is spin group 0 ++ ... ++ spin
 *     group n_spin-1 (head position j = i*batch + b); the tails of head i are
 *     the other spin groups in ascending order, then every categorical group;
 *     the weights are tiled n_spin times (row b for every i);
 *   - for each categorical group h, a group with head group h (j = b), tails
 *     every spin group, then the other categorical group; the weights with
 *     the head's category axis moved first (discrete_ebm.rs:493-540).
 * Slots (BlockSamplingProgram::new, crates/thrml-samplers/src/program.rs:102-
 * 200): for each free position, the groups in order and, inside a group, the
 * head positions j holding that node in ascending order.
 * Conditionals:
 *   SpinGibbsConditional::compute_parameters (crates/thrml-samplers/src/
 *   spin_gibbs.rs:512-595): gamma = 0, then per group gamma = gamma + (sum of
 *   the group's slots); a slot contributes w * prod(2 s_t - 1) over its spin
 *   tails, w = row b of the weights flattened to d1*d2 entries at index x (the
 *   state of the FIRST categorical tail, :553-575) or index 0 without one;
 *   s' = (u <= sigmoid(2 gamma)) (spin_gibbs.rs:95-97).
 *   CategoricalGibbsConditional::compute_parameters (crates/thrml-samplers/
 *   src/softmax.rs:586-710): theta[c] = 0, then per group theta[c] = theta[c]
 *   + (sum of the group's slots); a slot contributes prod(2 s_t - 1) * W'[c]
 *   without a categorical tail (W' = row b, d1*d2 = q entries), or
 *   prod(...) * W'[c][x] with the categorical tail x (W' = row b with the
 *   head axis first, [q][q]); x' = first argmax_c(theta[c] + Gumbel)
 *   (softmax.rs:60-97).
 * Uniforms (build convention shared with orc_ising.c / orc_potts.c): block
 * key k, block-local site i: spins take word i, categories word i*q + c of
 * ChaCha8Rng::seed_from_u64(k).  Sweeps follow sample_blocks / run_blocks
 * (crates/thrml-samplers/src/sampling.rs:28-106) with superblocks.
 * Energy: DiscreteEBMFactor::factor_energy (discrete_ebm.rs:551-593),
 * E = -sum_f sum_b W[b][x_c0][x_c1] prod(2 s - 1), accumulated in double.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "thrml_oracle.h"

typedef struct {
  uint32_t group;   /* interaction group index */
  size_t w_off;     /* row b of the factor's flat weights */
  int64_t cat_pos;  /* position of the first categorical tail, or -1 */
  uint32_t sc, sx;  /* categorical head: entry c * sc + x * sx of the row */
  uint32_t n_sp;    /* spin tails */
  size_t sp_beg;    /* first spin tail position in sp_pos */
} oslot;

typedef struct {
  uint32_t n_spin, n_cat, batch, d1, d2, square;
  uint32_t *nodes;
  size_t w_base;
} ofactor;

struct orc_discrete {
  uint32_t n_nodes, q, n_free, n_clamped;
  size_t n_total, n_free_total;
  uint32_t *blk_off, *pos_node;
  int64_t *node_pos;
  uint8_t *node_kind, *blk_kind;
  float *w;
  uint32_t n_factors;
  ofactor *f;
  size_t *slot_off;
  oslot *slots;
  uint32_t *sp_pos;
  uint32_t n_sb;
  uint32_t *sb_off;
};

static void set_err(char *err, size_t errlen, const char *msg) {
  if (err && errlen) snprintf(err, errlen, "%s", msg);
}

void orc_discrete_destroy(orc_discrete *p) {
  if (!p) return;
  free(p->blk_off);
  free(p->pos_node);
  free(p->node_pos);
  free(p->node_kind);
  free(p->blk_kind);
  free(p->w);
  if (p->f)
    for (uint32_t i = 0; i < p->n_factors; i++) free(p->f[i].nodes);
  free(p->f);
  free(p->slot_off);
  free(p->slots);
  free(p->sp_pos);
  free(p->sb_off);
  free(p);
}

/* the slot of head j of group `group` of factor fi, or -1 with err set when
 * a tail has no position */
static int make_slot(const orc_discrete *p, const ofactor *F, uint32_t group, int spin_head,
                     uint32_t head_i, uint32_t b, oslot *s, uint32_t *sp_out, char *err,
                     size_t errlen) {
  const uint32_t B = F->batch;
  s->group = group;
  s->w_off = F->w_base + (size_t)b * F->d1 * F->d2;
  s->cat_pos = -1;
  s->sc = 1;
  s->sx = 0;
  s->n_sp = 0;
  uint32_t n = 0;
  for (uint32_t k = 0; k < F->n_spin; k++) {
    if (spin_head && k == head_i) continue;
    const int64_t pos = p->node_pos[F->nodes[(size_t)k * B + b]];
    if (pos < 0) {
      set_err(err, errlen, "Node not found in global location map");
      return -1;
    }
    if (sp_out) sp_out[n] = (uint32_t)pos;
    n++;
  }
  s->n_sp = n;
  /* categorical tails: every categorical group for a spin head, the other
   * one for a categorical head; only the first is read (spin_gibbs.rs:
   * 553-575, softmax.rs:628-650), but every tail must have a position */
  for (uint32_t m = 0; m < F->n_cat; m++) {
    if (!spin_head && m == head_i) continue;
    const int64_t pos = p->node_pos[F->nodes[(size_t)(F->n_spin + m) * B + b]];
    if (pos < 0) {
      set_err(err, errlen, "Node not found in global location map");
      return -1;
    }
    if (s->cat_pos < 0) s->cat_pos = pos;
  }
  if (!spin_head) {
    if (s->cat_pos < 0) {
      s->sc = 1; /* W'[c]: the row's d1*d2 = q entries */
      s->sx = 0;
    } else if (head_i == 0) {
      s->sc = F->d2; /* W[b][c][x] */
      s->sx = 1;
    } else {
      s->sc = 1; /* W[b][x][c]: axes swapped (discrete_ebm.rs:523-534) */
      s->sx = F->d2;
    }
  }
  return 0;
}

orc_discrete *orc_discrete_create(uint32_t n_nodes, const uint8_t *node_kind, uint32_t q,
                                  uint32_t n_factors, const orc_factor *factors,
                                  uint32_t n_free, const uint32_t *free_off,
                                  const uint32_t *free_nodes, uint32_t n_clamped,
                                  const uint32_t *clamp_off, const uint32_t *clamp_nodes,
                                  char *err, size_t errlen) {
  orc_discrete *p = (orc_discrete *)calloc(1, sizeof(orc_discrete));
  p->n_nodes = n_nodes;
  p->q = q;
  p->n_free = n_free;
  p->n_clamped = n_clamped;
  p->node_kind = (uint8_t *)malloc((size_t)n_nodes + 1);
  int any_cat = 0;
  for (uint32_t x = 0; x < n_nodes; x++) {
    p->node_kind[x] = node_kind[x] ? 1 : 0;
    any_cat |= p->node_kind[x];
  }
  if (any_cat && (q < 2 || q > ORC_MAX_Q)) {
    set_err(err, errlen, "q must lie in 2..65536");
    orc_discrete_destroy(p);
    return NULL;
  }
  const uint32_t nb = n_free + n_clamped;
  p->blk_off = (uint32_t *)malloc((nb + 1) * sizeof(uint32_t));
  p->blk_kind = (uint8_t *)calloc(nb + 1, 1);
  p->blk_off[0] = 0;
  for (uint32_t b = 0; b < nb; b++) {
    const uint32_t len = b < n_free ? free_off[b + 1] - free_off[b]
                                    : clamp_off[b - n_free + 1] - clamp_off[b - n_free];
    if (len == 0) {
      set_err(err, errlen, "Encountered an empty block in BlockSpec");
      orc_discrete_destroy(p);
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
      const uint32_t node = b < n_free ? free_nodes[free_off[b] + (k - p->blk_off[b])]
                                       : clamp_nodes[clamp_off[b - n_free] + (k - p->blk_off[b])];
      if (node >= n_nodes) {
        set_err(err, errlen, "Node not found in global location map");
        orc_discrete_destroy(p);
        return NULL;
      }
      if (p->node_pos[node] >= 0) {
        set_err(err, errlen, "Node appears twice in blocks");
        orc_discrete_destroy(p);
        return NULL;
      }
      if (k > p->blk_off[b] && p->node_kind[node] != p->blk_kind[b]) {
        set_err(err, errlen, "a block holds both spin and categorical nodes");
        orc_discrete_destroy(p);
        return NULL;
      }
      p->blk_kind[b] = p->node_kind[node];
      p->node_pos[node] = (int64_t)k;
      p->pos_node[k] = node;
    }
  }

  /* factors: checks of DiscreteEBMFactor::new (discrete_ebm.rs:300-358) and
   * of what the two conditionals read */
  p->n_factors = n_factors;
  p->f = (ofactor *)calloc((size_t)n_factors + 1, sizeof(ofactor));
  size_t n_w = 0;
  for (uint32_t i = 0; i < n_factors; i++) {
    const orc_factor *F = &factors[i];
    const uint32_t ng = F->n_spin + F->n_cat;
    if (ng == 0) {
      set_err(err, errlen, "At least one node group must be provided");
      orc_discrete_destroy(p);
      return NULL;
    }
    if (F->n_cat > 2) {
      set_err(err, errlen, "weights are [b, d1, d2]: at most two categorical node groups");
      orc_discrete_destroy(p);
      return NULL;
    }
    if (F->batch == 0) {
      set_err(err, errlen, "Block cannot be empty");
      orc_discrete_destroy(p);
      return NULL;
    }
    if (F->d1 == 0 || F->d2 == 0) {
      set_err(err, errlen, "weight dimensions must be positive");
      orc_discrete_destroy(p);
      return NULL;
    }
    if (F->square && F->d1 != F->d2) {
      /* SquareDiscreteEBMFactor::new (discrete_ebm.rs:862-885) */
      set_err(err, errlen, "Interaction tensor is not square");
      orc_discrete_destroy(p);
      return NULL;
    }
    const uint32_t eff = F->d2 > 1 ? 2u : (F->d1 > 1 ? 1u : 0u); /* trailing 1s dropped */
    if (eff < F->n_cat) {
      char msg[256];
      snprintf(msg, sizeof msg,
               "The shape of the weight tensor must be [b, x_1, ..., x_k], where k is the "
               "length of categorical_node_groups (%u). Got effective dims: %u",
               F->n_cat, eff);
      set_err(err, errlen, msg);
      orc_discrete_destroy(p);
      return NULL;
    }
    for (uint32_t g = 0; g < ng; g++)
      for (uint32_t b = 0; b < F->batch; b++) {
        const uint32_t node = F->nodes[(size_t)g * F->batch + b];
        if (node >= n_nodes) {
          set_err(err, errlen, "Node not found in global location map");
          orc_discrete_destroy(p);
          return NULL;
        }
        if (p->node_kind[node] != (g >= F->n_spin)) {
          set_err(err, errlen,
                  "spin node groups must hold spin nodes and categorical node groups "
                  "categorical nodes");
          orc_discrete_destroy(p);
          return NULL;
        }
      }
    const uint32_t d = F->d1 * F->d2;
    if (F->n_spin && F->n_cat == 0 && d != 1) {
      set_err(err, errlen, "a spin factor without categorical groups has weights [b, 1, 1]");
      orc_discrete_destroy(p);
      return NULL;
    }
    if (F->n_spin && F->n_cat && d < q) {
      set_err(err, errlen, "a spin head indexes its weight row by a category: d1 * d2 >= q");
      orc_discrete_destroy(p);
      return NULL;
    }
    if (F->n_cat == 1 && d != q) {
      set_err(err, errlen, "a factor with one categorical group has weights [b, q, 1]");
      orc_discrete_destroy(p);
      return NULL;
    }
    if (F->n_cat == 2 && (F->d1 != q || F->d2 != q)) {
      set_err(err, errlen, "a factor with two categorical groups has weights [b, q, q]");
      orc_discrete_destroy(p);
      return NULL;
    }
    ofactor *o = &p->f[i];
    o->n_spin = F->n_spin;
    o->n_cat = F->n_cat;
    o->batch = F->batch;
    o->d1 = F->d1;
    o->d2 = F->d2;
    o->square = F->square;
    o->nodes = (uint32_t *)malloc((size_t)ng * F->batch * sizeof(uint32_t));
    memcpy(o->nodes, F->nodes, (size_t)ng * F->batch * sizeof(uint32_t));
    o->w_base = n_w;
    n_w += (size_t)F->batch * d;
  }
  p->w = (float *)malloc((n_w + 1) * sizeof(float));
  for (uint32_t i = 0; i < n_factors; i++)
    memcpy(p->w + p->f[i].w_base, factors[i].w,
           (size_t)factors[i].batch * factors[i].d1 * factors[i].d2 * sizeof(float));

  /* slots: a counting pass, then a filling pass in group order, head
   * position j ascending */
  const size_t nf = p->n_free_total;
  p->slot_off = (size_t *)calloc(nf + 2, sizeof(size_t));
  size_t n_sp_total = 0;
  for (int pass = 0; pass < 2; pass++) {
    size_t *fill = NULL;
    if (pass == 1) {
      for (size_t k = 0; k < nf; k++) p->slot_off[k + 1] += p->slot_off[k];
      p->slots = (oslot *)calloc(p->slot_off[nf] + 1, sizeof(oslot));
      p->sp_pos = (uint32_t *)malloc((n_sp_total + 1) * sizeof(uint32_t));
      fill = (size_t *)malloc((nf + 1) * sizeof(size_t));
      memcpy(fill, p->slot_off, (nf + 1) * sizeof(size_t));
      n_sp_total = 0;
    }
    uint32_t group = 0;
    for (uint32_t i = 0; i < n_factors; i++) {
      const ofactor *F = &p->f[i];
      const uint32_t n_heads = F->n_spin ? 1u + F->n_cat : F->n_cat;
      for (uint32_t hg = 0; hg < n_heads; hg++, group++) {
        const int spin_head = F->n_spin && hg == 0;
        const uint32_t h = F->n_spin ? hg - 1 : hg; /* categorical head group */
        /* merge_interaction_groups (discrete_ebm.rs:909-986) joins groups of
         * equal (tail count, spin tail count): in a square factor, the two
         * categorical-head groups */
        const uint32_t gid = F->square && !spin_head && h == 1 ? group - 1 : group;
        const uint32_t n_j = spin_head ? F->n_spin * F->batch : F->batch;
        for (uint32_t j = 0; j < n_j; j++) {
          const uint32_t hi = spin_head ? j / F->batch : h;
          const uint32_t b = spin_head ? j % F->batch : j;
          const uint32_t node = F->nodes[(size_t)(spin_head ? hi : F->n_spin + h) * F->batch + b];
          const int64_t pos = p->node_pos[node];
          if (pos < 0 || (size_t)pos >= nf) continue;
          oslot s;
          uint32_t *sp = pass == 1 ? p->sp_pos + n_sp_total : NULL;
          if (make_slot(p, F, gid, spin_head, hi, b, &s, sp, err, errlen)) {
            free(fill);
            orc_discrete_destroy(p);
            return NULL;
          }
          s.sp_beg = n_sp_total;
          n_sp_total += s.n_sp;
          if (pass == 0) {
            p->slot_off[pos + 1]++;
          } else {
            p->slots[fill[pos]++] = s;
          }
        }
      }
    }
    free(fill);
  }
  p->sb_off = orc_sb_partition(n_free, 0, NULL, &p->n_sb, NULL, 0);
  return p;
}

int orc_discrete_set_superblocks(orc_discrete *p, uint32_t n_sb, const uint32_t *off, char *err,
                                 size_t errlen) {
  uint32_t n = 0;
  uint32_t *r = orc_sb_partition(p->n_free, n_sb, off, &n, err, errlen);
  if (!r) return -1;
  free(p->sb_off);
  p->sb_off = r;
  p->n_sb = n;
  return 0;
}

size_t orc_discrete_total(const orc_discrete *p) { return p->n_total; }
int64_t orc_discrete_pos(const orc_discrete *p, uint32_t node) {
  return node < p->n_nodes ? p->node_pos[node] : -1;
}

static float spin_prod(const orc_discrete *p, const oslot *s, const uint16_t *st) {
  float sp = 1.0f;
  for (uint32_t t = 0; t < s->n_sp; t++) sp = sp * (st[p->sp_pos[s->sp_beg + t]] ? 1.0f : -1.0f);
  return sp;
}

/* gamma of spin position k */
static float spin_gamma(const orc_discrete *p, size_t k, const uint16_t *st) {
  float g = 0.0f, acc = 0.0f;
  for (size_t a = p->slot_off[k]; a < p->slot_off[k + 1]; a++) {
    const oslot *s = &p->slots[a];
    const uint32_t x = s->cat_pos >= 0 ? st[s->cat_pos] : 0u;
    const float v = p->w[s->w_off + x] * spin_prod(p, s, st);
    if (a == p->slot_off[k] || s->group != p->slots[a - 1].group) {
      if (a != p->slot_off[k]) g = g + acc;
      acc = v;
    } else {
      acc = acc + v;
    }
  }
  if (p->slot_off[k + 1] > p->slot_off[k]) g = g + acc;
  return g;
}

/* theta[0..q) of categorical position k; acc: q floats of scratch */
static void cat_theta(const orc_discrete *p, size_t k, const uint16_t *st, float *th, float *acc) {
  const uint32_t q = p->q;
  for (uint32_t c = 0; c < q; c++) th[c] = 0.0f;
  for (size_t a = p->slot_off[k]; a < p->slot_off[k + 1]; a++) {
    const oslot *s = &p->slots[a];
    const uint32_t x = s->cat_pos >= 0 ? st[s->cat_pos] : 0u;
    const float sp = spin_prod(p, s, st);
    const int first = a == p->slot_off[k] || s->group != p->slots[a - 1].group;
    if (first && a != p->slot_off[k])
      for (uint32_t c = 0; c < q; c++) th[c] = th[c] + acc[c];
    for (uint32_t c = 0; c < q; c++) {
      const float v = sp * p->w[s->w_off + (size_t)c * s->sc + (size_t)x * s->sx];
      acc[c] = first ? v : acc[c] + v;
    }
  }
  if (p->slot_off[k + 1] > p->slot_off[k])
    for (uint32_t c = 0; c < q; c++) th[c] = th[c] + acc[c];
}

void orc_discrete_params(const orc_discrete *p, const uint16_t *state, float *out) {
  const uint32_t qs = p->q > 1 ? p->q : 1;
  float *acc = (float *)malloc((size_t)qs * sizeof(float));
  for (uint32_t b = 0; b < p->n_free; b++)
    for (size_t k = p->blk_off[b]; k < p->blk_off[b + 1]; k++) {
      if (p->blk_kind[b])
        cat_theta(p, k, state, out + k * qs, acc);
      else
        out[k * qs] = spin_gamma(p, k, state);
    }
  free(acc);
}

/* block b of one chain from the state st, new values into tmp[0..n_b);
 * th: 2q floats of scratch */
static uint64_t block_update(const orc_discrete *p, uint32_t b, const uint32_t k8[8],
                             const uint16_t *st, uint16_t *tmp, float *th) {
  const uint32_t off = p->blk_off[b], n = p->blk_off[b + 1] - off;
  uint32_t blk[16];
  uint64_t cur = (uint64_t)-1, near = 0;
  if (!p->blk_kind[b]) {
    for (uint32_t i = 0; i < n; i++) {
      if ((i >> 4) != cur) {
        cur = i >> 4;
        orc_chacha_block(k8, cur, 0, 8, blk);
      }
      const float g = spin_gamma(p, off + i, st);
      const float prob = orc_sigmoid(g * 2.0f);
      const float u = (float)(blk[i & 15u] >> 8) * 0x1p-24f;
      tmp[i] = (uint16_t)(u <= prob);
      if (u > 0.0f && fabs(2.0 * (double)g - log((double)u / (1.0 - (double)u))) < 1e-5) near++;
    }
    return near;
  }
  const uint32_t q = p->q;
  for (uint32_t i = 0; i < n; i++) {
    cat_theta(p, off + i, st, th, th + q);
    float best = 0.0f, second = -INFINITY;
    uint32_t arg = 0;
    for (uint32_t c = 0; c < q; c++) {
      const uint64_t w = (uint64_t)i * q + c;
      if ((w >> 4) != cur) {
        cur = w >> 4;
        orc_chacha_block(k8, cur, 0, 8, blk);
      }
      const float v = th[c] + orc_gumbel(blk[w & 15]);
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
    if ((double)best - (double)second < 1e-5) near++;
  }
  return near;
}

static size_t max_superblock(const orc_discrete *p) {
  size_t m = 0;
  for (uint32_t s = 0; s < p->n_sb; s++) {
    const size_t l = p->blk_off[p->sb_off[s + 1]] - p->blk_off[p->sb_off[s]];
    if (l > m) m = l;
  }
  return m;
}

/* run_blocks of one chain (sampling.rs:81-106): sweep s keyed by
 * ckey.split(n_iters)[s], block b by sweep_key.split(n_free)[b]; superblocks
 * in order, each block of one reading the state from before it */
static uint64_t run_chain(const orc_discrete *p, uint64_t ckey, uint16_t *st, uint64_t n_iters,
                          uint16_t *tmp) {
  if (n_iters == 0) return 0;
  uint64_t near = 0;
  uint64_t *sk = (uint64_t *)malloc(n_iters * sizeof(uint64_t));
  uint64_t *bk = (uint64_t *)malloc((p->n_free + 1) * sizeof(uint64_t));
  float *th = (float *)malloc(2 * ((size_t)p->q + 1) * sizeof(float));
  orc_rng_split(ckey, n_iters, sk);
  for (uint64_t s = 0; s < n_iters; s++) {
    orc_rng_split(sk[s], p->n_free, bk);
    for (uint32_t g = 0; g < p->n_sb; g++) {
      const uint32_t first = p->sb_off[g], end = p->sb_off[g + 1];
      if (first == end) continue;
      const uint32_t base = p->blk_off[first];
      for (uint32_t b = first; b < end; b++) {
        uint32_t k8[8];
        orc_seed_from_u64(bk[b], k8);
        near += block_update(p, b, k8, st, tmp + (p->blk_off[b] - base), th);
      }
      memcpy(st + base, tmp, (p->blk_off[end] - base) * sizeof(uint16_t));
    }
  }
  free(th);
  free(sk);
  free(bk);
  return near;
}

void orc_discrete_run_blocks(const orc_discrete *p, uint64_t key, uint32_t C, uint16_t *state,
                             uint64_t n_iters, int n_threads, uint64_t *thr_sites) {
  uint64_t *ck = (uint64_t *)malloc(((size_t)C + 1) * sizeof(uint64_t));
  orc_rng_split(key, C, ck);
  const size_t maxb = max_superblock(p);
  uint64_t near = 0;
#pragma omp parallel for schedule(dynamic, 1) num_threads(n_threads > 0 ? n_threads : 1) reduction(+ : near)
  for (int64_t c = 0; c < (int64_t)C; c++) {
    uint16_t *tmp = (uint16_t *)malloc((maxb + 1) * sizeof(uint16_t));
    near += run_chain(p, ck[c], state + (size_t)c * p->n_total, n_iters, tmp);
    free(tmp);
  }
  free(ck);
  if (thr_sites) *thr_sites = near;
}

/* sample_states with every node observed (sampling.rs:128-156,178-320): the
 * key tree of orc_sample_states; out[n_obs][C][n_total], n_obs = max(n_samples, 1) */
void orc_discrete_sample_states(const orc_discrete *p, uint64_t key, orc_schedule sched,
                                uint32_t C, uint16_t *state, uint16_t *out, int n_threads) {
  const uint64_t n_obs = sched.n_samples > 1 ? sched.n_samples : 1;
  uint64_t *ck = (uint64_t *)malloc(((size_t)C + 1) * sizeof(uint64_t));
  orc_rng_split(key, C, ck);
  const size_t maxb = max_superblock(p);
#pragma omp parallel for schedule(dynamic, 1) num_threads(n_threads > 0 ? n_threads : 1)
  for (int64_t c = 0; c < (int64_t)C; c++) {
    uint16_t *st = state + (size_t)c * p->n_total;
    uint16_t *tmp = (uint16_t *)malloc((maxb + 1) * sizeof(uint16_t));
    uint64_t wk_sk[2];
    orc_rng_split(ck[c], 2, wk_sk);
    run_chain(p, wk_sk[0], st, sched.n_warmup, tmp);
    memcpy(out + (size_t)c * p->n_total, st, p->n_total * sizeof(uint16_t));
    if (n_obs > 1) {
      const uint64_t m = n_obs - 1;
      uint64_t *keys = (uint64_t *)malloc(m * sizeof(uint64_t));
      orc_rng_split(wk_sk[1], m, keys);
      for (uint64_t i = 0; i < m; i++) {
        run_chain(p, keys[i], st, sched.steps_per_sample, tmp);
        memcpy(out + ((size_t)(i + 1) * C + c) * p->n_total, st, p->n_total * sizeof(uint16_t));
      }
      free(keys);
    }
    free(tmp);
  }
  free(ck);
}

/* factor_energy of every factor from the raw factor definitions (not the
 * slots), summed: E = -sum_f sum_b W[b][x_c0][x_c1] prod(2 s - 1).  Factor
 * rows with a node outside every block are skipped. */
void orc_discrete_energy(const orc_discrete *p, uint32_t C, const uint16_t *state, double *out) {
  for (uint32_t c = 0; c < C; c++) {
    const uint16_t *st = state + (size_t)c * p->n_total;
    double e = 0.0;
    for (uint32_t i = 0; i < p->n_factors; i++) {
      const ofactor *F = &p->f[i];
      const uint32_t ng = F->n_spin + F->n_cat;
      for (uint32_t b = 0; b < F->batch; b++) {
        double sp = 1.0;
        size_t x0 = 0, x1 = 0;
        int skip = 0;
        for (uint32_t g = 0; g < ng; g++) {
          const int64_t pos = p->node_pos[F->nodes[(size_t)g * F->batch + b]];
          if (pos < 0) {
            skip = 1;
            break;
          }
          if (g < F->n_spin)
            sp *= st[pos] ? 1.0 : -1.0;
          else if (g == F->n_spin)
            x0 = st[pos];
          else
            x1 = st[pos];
        }
        if (skip) continue;
        /* one categorical group: entry x of the row's q entries; two:
         * W[b][x0][x1] */
        const size_t idx = F->n_cat == 2 ? x0 * F->d2 + x1 : x0;
        e += (double)p->w[F->w_base + (size_t)b * F->d1 * F->d2 + idx] * sp;
      }
    }
    out[c] = -e;
  }
}
