/*
 * orc_rbm.c -- oracle for the dense bipartite (RBM-shaped) Ising half-sweep.
 *
 * TEST INFRASTRUCTURE ONLY (see thrml_oracle.h).
 *
 * The reference has no dense path: an RBM is an IsingEBM whose edge list is
 * the complete bipartite graph (crates/thrml-models/src/ising.rs:26-143),
 * executed as a padded-ELL gather (crates/thrml-samplers/src/program.rs:114-230).
 * With the canonical edge order e = v*H + h over edges (v, V+h), the slot
 * order of hidden node h is v ascending and of visible node v is h ascending
 * (program.rs:102-200), so
 *   gamma_h = beta*c_h + sum_v (beta*W_vh)(2 s_v - 1),
 *   gamma_v = beta*b_v + sum_h (beta*W_vh)(2 s_h - 1).
 * The GPU evaluates the sums with matrix-core accumulation, whose order no
 * sequential restatement reproduces; this oracle sums the exact products in
 * double precision and rounds gamma once to f32, and flags (near[]) the
 * updates whose 2*gamma lies within `tol` of logit(u), where any two
 * summation orders may legitimately disagree.
 */
#include <math.h>
#include <stdlib.h>

#include "thrml_oracle.h"

void orc_rbm_half_sweep(uint32_t V, uint32_t H, const float *W, const float *bv,
                        const float *bh, float beta, uint32_t C,
                        const uint32_t *key8, int blk, uint8_t *sv, uint8_t *sh,
                        uint8_t *near, double tol, int n_threads) {
  const uint32_t n = blk == 0 ? V : H;
  /* the hidden update reads column i of W: a transposed copy makes it a
     contiguous row (the sum's order, v ascending, is unchanged) */
  float *Wt = NULL;
  if (blk != 0) {
    Wt = (float *)malloc((size_t)V * H * sizeof(float));
    for (uint32_t v = 0; v < V; v++)
      for (uint32_t h = 0; h < H; h++) Wt[(size_t)h * V + v] = W[(size_t)v * H + h];
  }
#pragma omp parallel for schedule(dynamic, 1) num_threads(n_threads > 0 ? n_threads : 1)
  for (int64_t c = 0; c < (int64_t)C; c++) {
    const uint32_t *k8 = key8 + (size_t)c * 8;
    uint8_t *out = blk == 0 ? sv + (size_t)c * V : sh + (size_t)c * H;
    const uint8_t *other = blk == 0 ? sh + (size_t)c * H : sv + (size_t)c * V;
    uint8_t *tmp = (uint8_t *)malloc(n);
    uint32_t words[16];
    for (uint32_t i = 0; i < n; i++) {
      double acc = 0.0;
      if (blk == 0) {
        for (uint32_t h = 0; h < H; h++) {
          float w = beta * W[(size_t)i * H + h];
          acc += other[h] ? (double)w : -(double)w;
        }
      } else {
        const float *col = Wt + (size_t)i * V;
        for (uint32_t v = 0; v < V; v++) {
          float w = beta * col[v];
          acc += other[v] ? (double)w : -(double)w;
        }
      }
      float bias = beta * (blk == 0 ? bv[i] : bh[i]);
      float g = (float)((double)bias + acc);
      if ((i & 15u) == 0) orc_chacha_block(k8, i >> 4, 0, 8, words);
      float u = (float)(words[i & 15u] >> 8) * 0x1p-24f;
      float prob = orc_sigmoid(g * 2.0f);
      tmp[i] = (uint8_t)(u <= prob);
      if (near) {
        double lu = u > 0.0f ? log((double)u / (1.0 - (double)u)) : -INFINITY;
        near[(size_t)c * n + i] = (uint8_t)(fabs(2.0 * ((double)bias + acc) - lu) < tol);
      }
    }
    for (uint32_t i = 0; i < n; i++) out[i] = tmp[i];
    free(tmp);
  }
  free(Wt);
}
