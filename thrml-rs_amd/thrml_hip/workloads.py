"""Synthetic inputs of the five benchmark configurations (and of the mixed
discrete-factor model the bench reports beside them).

Parameters come from the ChaCha8 stream of seed_from_u64(seed) through
Box-Muller (thrml_param_normal): biases use seed 1000 + config number, edge
couplings seed 1100 + config number.  The Erdos-Renyi graph of config 3 uses
seed 2003.  All sizes are the configurations' own.
"""
import numpy as np

from . import (Block, CategoricalEBMFactor, DiscreteEBMFactor, IsingEBM, SpinEBMFactor,
               SquareCategoricalEBMFactor, bf16_round, coloring_to_blocks, erdos_renyi,
               greedy_coloring, make_nearest_neighbor_lattice, param_normal)

CONFIGS = {
    1: dict(name="ising_lattice_64", L=64, chains=256, sweeps=1000, b_std=0.1, j_mean=0.3,
            j_std=0.05, beta=1.0, key=42),
    2: dict(name="ising_lattice_1024", L=1024, chains=64, sweeps=500, b_std=0.1, j_mean=0.44,
            j_std=0.05, beta=1.0, key=42),
    3: dict(name="ising_er_1m", N=1_000_000, mean_degree=12.0, chains=32, sweeps=200, b_std=0.2,
            j_mean=0.0, j_std=0.3, beta=1.0, key=42),
    4: dict(name="potts_lattice_512_q8", L=512, q=8, chains=32, sweeps=200, w_std=0.2,
            b_std=0.1, key=42),
    5: dict(name="rbm_1024x4096", V=1024, H=4096, chains=4096, sweeps=200, w_std=0.01,
            b_std=0.01, beta=1.0, key=42),
}


def lattice_ising(L, b_std, j_mean, j_std, beta=1.0, cfg=1, torus=True):
    """(IsingEBM, [upper, lower]) on the L x L periodic lattice."""
    n, edges, up, lo = make_nearest_neighbor_lattice(L, torus)
    b = param_normal(1000 + cfg, n, 0.0, b_std)
    w = param_normal(1100 + cfg, edges.shape[0], j_mean, j_std)
    return IsingEBM(n, edges, b, w, beta), [up, lo]


def config_ising(cfg, L=None):
    c = CONFIGS[cfg]
    return lattice_ising(L or c["L"], c["b_std"], c["j_mean"], c["j_std"], c["beta"], cfg)


def er_ising(N, mean_degree, b_std, j_mean, j_std, beta=1.0, cfg=3):
    p = mean_degree / (N - 1)
    edges = erdos_renyi(N, p, 2000 + cfg)
    color = greedy_coloring(N, edges)
    blocks = coloring_to_blocks(color)
    b = param_normal(1000 + cfg, N, 0.0, b_std)
    w = param_normal(1100 + cfg, edges.shape[0], j_mean, j_std)
    return IsingEBM(N, edges, b, w, beta), blocks


def config3(N=None):
    c = CONFIGS[3]
    return er_ising(N or c["N"], c["mean_degree"], c["b_std"], c["j_mean"], c["j_std"], c["beta"])


def potts_lattice(L, q, w_std, b_std, cfg=4):
    n, edges, up, lo = make_nearest_neighbor_lattice(L, True)
    W = param_normal(1100 + cfg, edges.shape[0] * q * q, 0.0, w_std).reshape(-1, q, q)
    bias = param_normal(1000 + cfg, n * q, 0.0, b_std).reshape(n, q)
    return n, edges, W, bias, [up, lo]


def rbm(V, H, w_std, b_std, cfg=5):
    W = param_normal(1100 + cfg, V * H, 0.0, w_std).reshape(V, H)
    bits, Wf = bf16_round(W)
    bv = param_normal(1000 + cfg, V, 0.0, b_std)
    bh = param_normal(1200 + cfg, H, 0.0, b_std)
    return bits, Wf, bv, bh


def rbm_f32(V, H, w_std, b_std, cfg=5):
    """Config 5's RBM with its weights kept in f32 (the reference's IsingEBM
    type): (W, bv, bh)."""
    W = param_normal(1100 + cfg, V * H, 0.0, w_std).reshape(V, H)
    bv = param_normal(1000 + cfg, V, 0.0, b_std)
    bh = param_normal(1200 + cfg, H, 0.0, b_std)
    return W, bv, bh


def algorithmic_bytes(cfg, n_nodes, n_edges, chains, q=8):
    """B_alg per sweep: int8 state read + written once per chain, parameters
    once, indices implicit (lattice) or one i32 per directed slot (CSR)."""
    if cfg in (1, 2):
        return 2 * chains * n_nodes + 4 * n_nodes + 4 * n_edges
    if cfg == 3:
        return 2 * chains * n_nodes + 4 * n_nodes + 2 * n_edges * 8
    if cfg == 4:
        return 2 * chains * n_nodes + 4 * q * n_nodes + 4 * q * q * n_edges
    raise ValueError(cfg)


def rbm_flops(V, H, chains):
    return 4 * chains * V * H


def mixed_lattice(L, q):
    """A 2-layer torus: spins S (node i) and q-state categorical nodes X
    (node L^2 + i), with spin biases and couplings, categorical biases and
    square pair factors, and a spin-categorical factor per site; blocks are
    the two checkerboard halves of each layer."""
    n, edges, up, lo = make_nearest_neighbor_lattice(L, True)
    rng = np.random.default_rng(77)
    S = np.arange(n, dtype=np.uint32)
    X = S + n
    eu, ev = edges[:, 0].astype(np.uint32), edges[:, 1].astype(np.uint32)
    E = eu.size
    fs = [SpinEBMFactor([S], rng.normal(0, 0.2, (n, 1, 1)).astype(np.float32)),
          SpinEBMFactor([eu, ev], rng.normal(0.3, 0.1, (E, 1, 1)).astype(np.float32)),
          CategoricalEBMFactor([X], rng.normal(0, 0.3, (n, q, 1)).astype(np.float32)),
          SquareCategoricalEBMFactor([X[eu], X[ev]],
                                     rng.normal(0, 0.3, (E, q, q)).astype(np.float32)),
          DiscreteEBMFactor([S], [X], rng.normal(0, 0.3, (n, q, 1)).astype(np.float32))]
    kinds = np.r_[np.zeros(n), np.ones(n)].astype(np.uint8)
    blocks = [up.nodes, lo.nodes, up.nodes + n, lo.nodes + n]
    return 2 * n, kinds, fs, blocks
