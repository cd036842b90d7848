"""Pins of the oracle's Ising sweep that do not retype its formula.

  - gamma by the energy-difference identity: gamma_i = -(E(s_i=+1) - E(s_i=-1))/2
    with E from IsingEBM::energy (crates/thrml-models/src/ising.rs:151-222),
    which the oracle evaluates from the raw edge list, not from the slots;
  - closed forms: isolated spins <s> = tanh(beta b); zero-field open chain
    <s_i s_i+1> = tanh(beta J);
  - exact enumeration (the reference's dead-code utility
    crates/thrml-models/tests/utils.rs:202-335 revived): moments of a 3x4
    open lattice against the exact Boltzmann sums;
  - hinton_init statistics (crates/thrml-models/tests/test_ising.rs:58-98);
  - structure: run_blocks(n_iters = 0) is the identity (sampling.rs:89-91);
    error strings of BlockSpec::new (blockspec.rs:36-54).
A planted mistake (sigmoid(gamma) instead of sigmoid(2 gamma), or u >= p)
moves the moments by more than ten standard errors.
"""
import itertools

import numpy as np
import pytest

import pyoracle as orc


def _rand_graph(n, m, seed):
    rng = np.random.default_rng(seed)
    e = set()
    while len(e) < m:
        a, b = rng.integers(0, n, 2)
        if a != b:
            e.add((int(a), int(b)))  # arbitrary orientation: u may exceed v
    return np.array(sorted(e), dtype=np.uint32)


def test_gamma_energy_difference_identity():
    n = 40
    edges = _rand_graph(n, 120, 1)
    rng = np.random.default_rng(2)
    b = rng.normal(0, 0.5, n).astype(np.float32)
    w = rng.normal(0, 0.7, edges.shape[0]).astype(np.float32)
    beta = 0.8
    perm = rng.permutation(n)
    blocks = [perm[:13], perm[13:29], perm[29:]]
    p = orc.Ising(n, edges, b, w, beta, blocks)
    st = rng.integers(0, 2, (1, p.n_total)).astype(np.uint8)
    gam = p.gamma(st[0])
    k = 0
    for blk in blocks:
        for node in blk:
            pos = p.pos(node)
            up = st.copy()
            up[0, pos] = 1
            dn = st.copy()
            dn[0, pos] = 0
            de = p.energy(up)[0] - p.energy(dn)[0]
            assert abs(gam[k] - (-de / 2)) < 1e-4 * (1 + abs(de)), (node, gam[k], de)
            k += 1


def test_energy_reference_cases():
    """The reference's energy tests (crates/thrml-models/tests/test_ising.rs:139-212)
    with their values worked by hand: a 3-node chain, b = (0.1, 0.2, 0.3),
    J = (0.5, -0.5), four states; a 4-node chain, b = 0, J = 1, state 1010."""
    p = orc.Ising(3, [(0, 1), (1, 2)], np.array([0.1, 0.2, 0.3], np.float32),
                  np.array([0.5, -0.5], np.float32), 1.0, [[0, 1, 2]])
    st = np.array([[0, 0, 0], [1, 1, 1], [1, 0, 1], [0, 1, 0]], np.uint8)
    assert np.allclose(p.energy(st), [0.6, -0.6, -0.2, 0.2], atol=1e-6)
    p = orc.Ising(4, [(0, 1), (1, 2), (2, 3)], np.zeros(4, np.float32),
                  np.ones(3, np.float32), 1.0, [[0, 1, 2, 3]])
    assert np.allclose(p.energy(np.array([[1, 0, 1, 0]], np.uint8)), [3.0])


def test_isolated_spins_closed_form():
    n = 6
    b = np.array([-1.0, -0.3, 0.0, 0.2, 0.7, 1.5], np.float32)
    p = orc.Ising(n, np.zeros((0, 2), np.uint32), b, np.zeros(0, np.float32), 1.0,
                  [[0, 2, 4], [1, 3, 5]])
    C = 4096
    ns, es, _, _ = p.estimate_moments(7, (5, 200, 1), np.zeros((C, n), np.uint8), np.arange(n),
                                      np.zeros((0, 2)))
    m = ns / (C * 200)
    se = 1.0 / np.sqrt(C * 200)
    assert np.all(np.abs(m - np.tanh(b)) < 6 * se), (m, np.tanh(b))


def test_open_chain_correlation_closed_form():
    n = 8
    edges = np.array([[i, i + 1] for i in range(n - 1)], np.uint32)
    J = np.array([0.2, -0.4, 0.6, 0.1, -0.9, 0.3, 0.5], np.float32)
    p = orc.Ising(n, edges, np.zeros(n, np.float32), J, 1.0, [[0, 2, 4, 6], [1, 3, 5, 7]])
    C = 2048
    ns, es, _, _ = p.estimate_moments(11, (20, 400, 2), np.zeros((C, n), np.uint8), np.arange(n),
                                      edges)
    m2 = es / (C * 400)
    se = 2.0 / np.sqrt(C * 400)
    assert np.all(np.abs(m2 - np.tanh(J)) < 6 * se), (m2, np.tanh(J))
    assert np.all(np.abs(ns / (C * 400)) < 6 * se)


def test_exact_enumeration_moments():
    # 3 x 4 open lattice, random fields and couplings, checkerboard blocks
    R, Cc = 3, 4
    n = R * Cc
    e = []
    for r in range(R):
        for c in range(Cc):
            x = r * Cc + c
            if r + 1 < R:
                e.append((x, x + Cc))
            if c + 1 < Cc:
                e.append((x, x + 1))
    edges = np.array(e, np.uint32)
    rng = np.random.default_rng(4)
    b = rng.normal(0, 0.3, n).astype(np.float32)
    w = rng.normal(0.2, 0.4, edges.shape[0]).astype(np.float32)
    beta = 1.0
    blk0 = [x for x in range(n) if ((x // Cc) + (x % Cc)) % 2 == 0]
    blk1 = [x for x in range(n) if ((x // Cc) + (x % Cc)) % 2 == 1]
    # exact Boltzmann moments
    S = np.array(list(itertools.product([-1, 1], repeat=n)), np.float64)
    E = -beta * (S @ b.astype(np.float64) + (S[:, edges[:, 0]] * S[:, edges[:, 1]]) @ w.astype(np.float64))
    pr = np.exp(-(E - E.min()))
    pr /= pr.sum()
    m1 = pr @ S
    m2 = pr @ (S[:, edges[:, 0]] * S[:, edges[:, 1]])
    p = orc.Ising(n, edges, b, w, beta, [blk0, blk1])
    C, ns = 2048, 300
    init = np.zeros((C, p.n_total), np.uint8)
    s1, s2, _, _ = p.estimate_moments(3, (50, ns, 3), init, np.arange(n), edges)
    se = 1.0 / np.sqrt(C * ns)
    assert np.all(np.abs(s1 / (C * ns) - m1) < 8 * se), (s1 / (C * ns), m1)
    assert np.all(np.abs(s2 / (C * ns) - m2) < 8 * se)


def test_hinton_statistics():
    n = 10
    b = np.full(n, 10.0, np.float32)
    p = orc.Ising(n, np.zeros((0, 2), np.uint32), b, np.zeros(0, np.float32), 1.0, [np.arange(n)])
    st = p.hinton_init(5, 1)
    assert st.sum() >= 7  # test_ising.rs:58-98
    b = np.linspace(-2, 2, 50).astype(np.float32)
    p = orc.Ising(50, np.zeros((0, 2), np.uint32), b, np.zeros(0, np.float32), 0.5,
                  [np.arange(25), np.arange(25, 50)])
    st = p.hinton_init(9, 20000)
    frac = st.mean(axis=0)
    want = 1 / (1 + np.exp(-0.5 * b))
    assert np.all(np.abs(frac - want) < 6 * np.sqrt(want * (1 - want) / 20000))


def test_run_blocks_zero_iters_identity_and_errors():
    edges = np.array([[0, 1], [1, 2]], np.uint32)
    p = orc.Ising(3, edges, np.zeros(3, np.float32), np.ones(2, np.float32), 1.0, [[0, 2], [1]])
    st = np.array([[1, 0, 1]], np.uint8)
    out, _ = p.run_blocks(1, st, 0)
    assert np.array_equal(out, st)
    with pytest.raises(ValueError, match="twice"):
        orc.Ising(3, edges, np.zeros(3, np.float32), np.ones(2, np.float32), 1.0, [[0, 1], [1, 2]])
    with pytest.raises(ValueError, match="empty"):
        orc.Ising(3, edges, np.zeros(3, np.float32), np.ones(2, np.float32), 1.0, [[0, 1, 2], []])


def test_opbyop_baseline_equals_fused_oracle():
    # the timed op-by-op CPU baseline must compute the same trajectories
    n, edges, up, lo = 64, orc.lattice_edges(8, True), *orc.lattice_blocks(8)
    rng = np.random.default_rng(8)
    b = rng.normal(0, 0.1, 64).astype(np.float32)
    w = rng.normal(0.4, 0.05, edges.shape[0]).astype(np.float32)
    p = orc.Ising(64, edges, b, w, 1.0, [up, lo])
    init = p.hinton_init(1, 5)
    a, _ = p.run_blocks(42, init, 30)
    c = p.run_blocks_opbyop(42, init, 30)
    assert np.array_equal(a, c)


def test_sample_states_agrees_with_moment_run():
    """The oracle's sample_states (every node observed) and estimate_moments
    walk one key tree: summed over chains and observations, t = 2s - 1 of
    the samples gives the moment sums, and the last sample is the moment
    run's final state; observation 0 is the state after the warmup alone."""
    edges = _rand_graph(40, 90, 9)
    rng = np.random.default_rng(9)
    b = rng.normal(0, 0.4, 40).astype(np.float32)
    w = rng.normal(0, 0.5, edges.shape[0]).astype(np.float32)
    blocks = [np.arange(0, 40, 3), np.arange(1, 40, 3), np.arange(2, 40, 3)]
    p = orc.Ising(40, edges, b, w, 0.8, blocks)
    init = rng.integers(0, 2, (9, p.n_total)).astype(np.uint8)
    obs = p.sample_states(77, (3, 5, 2), init)
    assert obs.shape == (5, 9, p.n_total)
    pos = np.array([p.pos(x) for x in range(40)])
    ns, es, fin, _ = p.estimate_moments(77, (3, 5, 2), init, np.arange(40), edges)
    t = 2 * obs.astype(np.int64) - 1
    assert np.array_equal(t[:, :, pos].sum(axis=(0, 1)), ns)
    assert np.array_equal((t[:, :, pos[edges[:, 0]]] * t[:, :, pos[edges[:, 1]]]).sum(axis=(0, 1)), es)
    assert np.array_equal(obs[-1], fin)
    _, _, fin1, _ = p.estimate_moments(77, (3, 1, 2), init, np.arange(40), edges)
    assert np.array_equal(obs[0], fin1)
    assert np.array_equal(p.sample_states(77, (3, 0, 2), init)[0], fin1)
    assert not np.array_equal(obs[0], obs[-1])


def test_hinton_init_distribution():
    """hinton_init (crates/thrml-models/src/ising.rs:602-673) samples
    s_i = (u <= sigmoid(beta b_i)) with u from the backend's global
    Tensor::random; its key is split and unused (:618), so this build's keyed
    stream (block key split(n_blocks)[b], entry (c, i) = keystream word
    c n_b + i) is its own deterministic convention and parity with the
    reference is in distribution: every node's frequency over 20000 chains
    lies within 5 standard errors of sigmoid(beta b_i), the rate a planted
    sigmoid(2 beta b) or sigmoid(b) (beta dropped) misses by far more, and
    different keys give different draws."""
    import math

    n = 60
    rng = np.random.default_rng(8)
    edges = np.array([(i, i + 1) for i in range(n - 1)], np.uint32)
    b = rng.normal(0, 1.2, n).astype(np.float32)
    beta = 0.7
    o = orc.Ising(n, edges, b, np.zeros(n - 1, np.float32), beta, [np.arange(0, n, 2),
                                                                   np.arange(1, n, 2)])
    C = 20000
    st = o.hinton_init(11, C)
    freq = np.zeros(n)
    for node in range(n):
        freq[node] = st[:, o.pos(node)].mean()
    p = 1.0 / (1.0 + np.exp(-beta * b.astype(np.float64)))
    se = np.sqrt(p * (1 - p) / C)
    assert np.all(np.abs(freq - p) < 5 * se + 1e-12)
    for wrong in (1.0 / (1.0 + np.exp(-2 * beta * b)), 1.0 / (1.0 + np.exp(-b.astype(np.float64)))):
        z = np.abs(freq - wrong) / np.sqrt(wrong * (1 - wrong) / C)
        assert z.max() > 10
    assert not np.array_equal(o.hinton_init(12, 64), st[:64])
    assert math.isclose(float(st.mean()), float(p.mean()), abs_tol=0.01)
