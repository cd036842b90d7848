/*
 * orc_graph.c -- oracle graph builders and synthetic parameters.
 *
 * TEST INFRASTRUCTURE ONLY (see thrml_oracle.h).
 *
 * make_nearest_neighbor_lattice (crates/thrml-models/src/graph_utils.rs:177-243)
 * collects edges in a HashSet, so its edge order differs from process to
 * process.  The canonical order used by the build: visit idx = 0..size-1,
 * jumps (1,0) then (0,1), emit (min, max) unless already emitted.
 * greedy_coloring (crates/thrml-examples/src/lib.rs:114-147) assigns the
 * smallest colour unused by already-coloured neighbours, visiting nodes in
 * index order; coloring_to_blocks (lib.rs:186-205) groups nodes by colour
 * (HashMap order in the reference, ascending node id here).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "thrml_oracle.h"

size_t orc_lattice_edges(uint32_t side, int torus, uint32_t *u, uint32_t *v) {
  side = (side + 1) / 2 * 2; /* graph_utils.rs:184 rounds up to even */
  const int64_t L = side;
  const int64_t size = L * L;
  /* duplicates can only arise for side == 2 on a torus; a tiny set check */
  size_t ne = 0;
  uint32_t *tu = NULL, *tv = NULL;
  size_t cap = (size_t)size * 2;
  tu = (uint32_t *)malloc(cap * sizeof(uint32_t));
  tv = (uint32_t *)malloc(cap * sizeof(uint32_t));
  for (int64_t idx = 0; idx < size; idx++) {
    int64_t i = idx / L, j = idx % L;
    const int di[2] = {1, 0}, dj[2] = {0, 1};
    for (int t = 0; t < 2; t++) {
      int64_t ii = i + di[t], jj = j + dj[t];
      int64_t tgt;
      if (torus) {
        ii = ((ii % L) + L) % L;
        jj = ((jj % L) + L) % L;
        tgt = ii * L + jj;
      } else {
        if (ii < 0 || ii >= L || jj < 0 || jj >= L) continue;
        tgt = ii * L + jj;
      }
      uint32_t a = (uint32_t)(idx < tgt ? idx : tgt);
      uint32_t b = (uint32_t)(idx < tgt ? tgt : idx);
      int dup = 0;
      if (side <= 2) {
        for (size_t k = 0; k < ne; k++)
          if (tu[k] == a && tv[k] == b) dup = 1;
      }
      if (a == b) dup = 1; /* self loop impossible for side>=2; guard anyway */
      if (!dup) {
        tu[ne] = a;
        tv[ne] = b;
        ne++;
      }
    }
  }
  if (u && v) {
    memcpy(u, tu, ne * sizeof(uint32_t));
    memcpy(v, tv, ne * sizeof(uint32_t));
  }
  free(tu);
  free(tv);
  return ne;
}

void orc_lattice_blocks(uint32_t side, uint32_t *upper, uint32_t *lower) {
  side = (side + 1) / 2 * 2;
  size_t nu = 0, nl = 0;
  for (uint32_t idx = 0; idx < side * side; idx++) {
    uint32_t i = idx / side, j = idx % side;
    if (((i + j) & 1u) == 0)
      upper[nu++] = idx; /* graph_utils.rs:232 */
    else
      lower[nl++] = idx;
  }
}

uint32_t orc_greedy_coloring(uint32_t n, size_t n_edges, const uint32_t *u,
                             const uint32_t *v, uint32_t *color) {
  /* adjacency in CSR */
  size_t *off = (size_t *)calloc((size_t)n + 1, sizeof(size_t));
  for (size_t e = 0; e < n_edges; e++) {
    off[u[e] + 1]++;
    off[v[e] + 1]++;
  }
  for (uint32_t i = 0; i < n; i++) off[i + 1] += off[i];
  uint32_t *adj = (uint32_t *)malloc((off[n] + 1) * sizeof(uint32_t));
  size_t *fill = (size_t *)malloc(((size_t)n + 1) * sizeof(size_t));
  memcpy(fill, off, ((size_t)n + 1) * sizeof(size_t));
  for (size_t e = 0; e < n_edges; e++) {
    adj[fill[u[e]]++] = v[e];
    adj[fill[v[e]]++] = u[e];
  }
  uint32_t n_colors = 0;
  unsigned char *used = NULL;
  size_t used_cap = 0;
  for (uint32_t x = 0; x < n; x++) color[x] = UINT32_MAX;
  for (uint32_t x = 0; x < n; x++) {
    size_t deg = off[x + 1] - off[x];
    if (deg + 2 > used_cap) {
      used_cap = deg + 2;
      used = (unsigned char *)realloc(used, used_cap);
    }
    memset(used, 0, deg + 2);
    for (size_t k = off[x]; k < off[x + 1]; k++) {
      uint32_t c = color[adj[k]];
      if (c != UINT32_MAX && c <= deg) used[c] = 1;
    }
    uint32_t c = 0;
    while (used[c]) c++;
    color[x] = c;
    if (c + 1 > n_colors) n_colors = c + 1;
  }
  free(used);
  free(off);
  free(adj);
  free(fill);
  return n_colors;
}

void orc_param_normal(uint64_t seed, size_t n, double mean, double std, float *out) {
  /* u32 words w of the ChaCha8 stream of seed_from_u64(seed); pairs
   * (w0, w1) -> u = (w + 0.5) / 2^32 in (0,1);
   * z0 = sqrt(-2 ln u0) cos(2 pi u1), z1 = ... sin(...). */
  uint32_t k8[8], blk[16];
  orc_seed_from_u64(seed, k8);
  uint64_t widx = 0;
  uint64_t cur = (uint64_t)-1;
  const double two_pi = 6.283185307179586476925286766559;
  for (size_t i = 0; i < n; i += 2) {
    uint32_t w[2];
    for (int t = 0; t < 2; t++) {
      if ((widx >> 4) != cur) {
        cur = widx >> 4;
        orc_chacha_block(k8, cur, 0, 8, blk);
      }
      w[t] = blk[widx & 15];
      widx++;
    }
    double u0 = ((double)w[0] + 0.5) / 4294967296.0;
    double u1 = ((double)w[1] + 0.5) / 4294967296.0;
    double r = sqrt(-2.0 * log(u0));
    out[i] = (float)(mean + std * r * cos(two_pi * u1));
    if (i + 1 < n) out[i + 1] = (float)(mean + std * r * sin(two_pi * u1));
  }
}
