"""Pins of the oracle's categorical (Potts) sweep that do not retype its
formula (crates/thrml-samplers/src/softmax.rs:60-97,586-710,
crates/thrml-models/src/discrete_ebm.rs:456-548).

  - theta by the energy-difference identity: theta_n[c] - theta_n[0] =
    -(E(x_n = c) - E(x_n = 0)) with E(x) = -(sum_n b[n][x_n] + sum_e W[e][x_u][x_v])
    evaluated from the raw factor arrays (orientation of W in both roles);
  - exact enumeration: node and edge marginals of a 2 x 3 grid with q = 3
    against the exact Boltzmann distribution over all 3^6 states;
  - the reference's strong-logit test (softmax.rs:873-898): logits +-10 give
    categories 2 and 1; and at q = 40, where a site's words span several
    ChaCha8 blocks;
  - q = 20 (words across block boundaries): marginals of a 3-node chain
    against exact enumeration;
  - structure: empty blocks, unknown nodes and q outside 2..65536 are rejected.
A planted transposition of W in either role moves the marginals by more than
ten standard errors (checked here on the CPU).
"""
import itertools

import numpy as np
import pytest

import pyoracle as orc


def _energy(x, bias, eu, ev, W):
    e = sum(float(bias[n, x[n]]) for n in range(len(x)))
    e += sum(float(W[k, x[eu[k]], x[ev[k]]]) for k in range(len(eu)))
    return -e


@pytest.mark.parametrize("q", [5, 40, 256, 300])
def test_theta_energy_difference_identity(q):
    rng = np.random.default_rng(3 + q)
    n = 30
    edges = set()
    while len(edges) < 80:
        a, b = (int(v) for v in rng.integers(0, n, 2))
        if a != b:
            edges.add((a, b))  # arbitrary orientation: u may exceed v
    edges = np.array(sorted(edges), np.uint32)
    W = rng.normal(0, 0.8, (len(edges), q, q)).astype(np.float32)
    bias = rng.normal(0, 0.5, (n, q)).astype(np.float32)
    perm = rng.permutation(n)
    blocks = [perm[:11], perm[11:20], perm[20:]]
    p = orc.Potts(n, q, edges, W, bias, blocks)
    eu, ev = edges[:, 0], edges[:, 1]
    for trial in range(3 if q <= 40 else 1):
        x = rng.integers(0, q, n)
        glob = np.zeros(p.n_total, np.uint16)
        for node in range(n):
            glob[p.pos(node)] = x[node]
        th = p.theta(glob)
        for node in range(n):
            e0 = None
            for c in range(q):
                y = x.copy()
                y[node] = c
                e = _energy(y, bias, eu, ev, W)
                if c == 0:
                    e0, t0 = e, th[p.pos(node), 0]
                else:
                    assert abs((th[p.pos(node), c] - t0) - (-(e - e0))) < 2e-5


def test_oracle_energy_pinned_by_theta():
    """orc_potts_energy (the oracle's factor energies, from its edge list)
    against theta of the sweep code (from the slot lists): for every node and
    category, theta[c] - theta[0] = -(E(x_n = c) - E(x_n = 0)).  Asymmetric W
    in both roles, so a transposed W or a swapped endpoint fails."""
    rng = np.random.default_rng(11)
    n, q = 24, 4
    edges = set()
    while len(edges) < 60:
        a, b = (int(v) for v in rng.integers(0, n, 2))
        if a != b:
            edges.add((a, b))
    edges = np.array(sorted(edges), np.uint32)
    W = rng.normal(0, 0.8, (len(edges), q, q)).astype(np.float32)
    bias = rng.normal(0, 0.5, (n, q)).astype(np.float32)
    perm = rng.permutation(n)
    p = orc.Potts(n, q, edges, W, bias, [perm[:10], perm[10:]])
    x = rng.integers(0, q, p.n_total).astype(np.uint8)
    th = p.theta(x)
    for pos in range(p.n_total):
        ys = np.repeat(x[None, :], q, axis=0)
        ys[:, pos] = np.arange(q)
        e = p.energy(ys)
        assert np.allclose(th[pos] - th[pos, 0], -(e - e[0]), atol=2e-5), pos


def test_oracle_energy_hand_values():
    # two nodes, one edge (0, 1): E = -(b[0][x0] + b[1][x1] + W[x0][x1])
    bias = np.array([[0.1, 0.2], [0.3, 0.4]], np.float32)
    W = np.array([[[1.0, 2.0], [3.0, 4.0]]], np.float32)
    p = orc.Potts(2, 2, [(0, 1)], W, bias, [[0], [1]])
    st = np.array([[0, 0], [1, 0], [0, 1], [1, 1]], np.uint8)  # positions = nodes here
    want = -np.array([0.1 + 0.3 + 1.0, 0.2 + 0.3 + 3.0, 0.1 + 0.4 + 2.0, 0.2 + 0.4 + 4.0])
    assert np.allclose(p.energy(st), want, atol=1e-6)


def _grid_potts(W_scale=1.0, seed=5):
    rng = np.random.default_rng(seed)
    # 2 x 3 open grid, node = 3*r + c
    edges = np.array([(0, 1), (1, 2), (3, 4), (4, 5), (0, 3), (1, 4), (2, 5)], np.uint32)
    q = 3
    W = (W_scale * rng.normal(0, 0.9, (len(edges), q, q))).astype(np.float32)
    bias = rng.normal(0, 0.6, (6, q)).astype(np.float32)
    blocks = [np.array([0, 2, 4], np.uint32), np.array([1, 3, 5], np.uint32)]
    return edges, W, bias, blocks, q


def _exact_marginals(edges, W, bias, q, n=6):
    eu, ev = edges[:, 0], edges[:, 1]
    states = np.array(list(itertools.product(range(q), repeat=n)))
    E = np.array([_energy(s, bias, eu, ev, W) for s in states])
    pr = np.exp(-(E - E.min()))
    pr /= pr.sum()
    node = np.zeros((n, q))
    for s, w in zip(states, pr):
        node[np.arange(n), s] += w
    pair = np.zeros((len(edges), q, q))
    for k, (a, b) in enumerate(edges):
        for s, w in zip(states, pr):
            pair[k, s[a], s[b]] += w
    return node, pair


def _sampled_marginals(p, edges, q, C=20000, sweeps=25, key=11, n=6):
    st, _ = p.run_blocks(key, np.zeros((C, p.n_total), np.uint8), sweeps)
    x = np.zeros((C, n), np.int64)
    for node in range(n):
        x[:, node] = st[:, p.pos(node)]
    node = np.stack([(x == c).mean(0) for c in range(q)], axis=1)
    pair = np.zeros((len(edges), q, q))
    for k, (a, b) in enumerate(edges):
        for i in range(q):
            for j in range(q):
                pair[k, i, j] = ((x[:, a] == i) & (x[:, b] == j)).mean()
    return node, pair


def test_exact_enumeration_marginals():
    edges, W, bias, blocks, q = _grid_potts()
    exact_node, exact_pair = _exact_marginals(edges, W, bias, q)
    p = orc.Potts(6, q, edges, W, bias, blocks)
    node, pair = _sampled_marginals(p, edges, q)
    C = 20000
    se_node = np.sqrt(exact_node * (1 - exact_node) / C) + 1e-9
    se_pair = np.sqrt(exact_pair * (1 - exact_pair) / C) + 1e-9
    assert np.max(np.abs(node - exact_node) / se_node) < 5.0
    assert np.max(np.abs(pair - exact_pair) / se_pair) < 5.0


@pytest.mark.parametrize("mistake", ["transpose_u", "transpose_v"])
def test_planted_transposition_is_detected(mistake):
    """The oracle run on a model whose W is transposed for one role (emulating
    a role mix-up) disagrees with the exact marginals of the true model."""
    edges, W, bias, blocks, q = _grid_potts()
    exact_node, exact_pair = _exact_marginals(edges, W, bias, q)
    # a role mix-up is equivalent to swapping the endpoints of every edge while
    # keeping W: W[e][x_v][x_u] instead of W[e][x_u][x_v]
    bad_edges = edges[:, ::-1].copy() if mistake == "transpose_u" else edges
    bad_W = W if mistake == "transpose_u" else np.ascontiguousarray(W.transpose(0, 2, 1))
    p = orc.Potts(6, q, bad_edges, bad_W, bias, blocks)
    node, pair = _sampled_marginals(p, bad_edges, q)
    if mistake == "transpose_u":
        pair = pair.transpose(0, 2, 1)
    se = np.sqrt(exact_pair * (1 - exact_pair) / 20000) + 1e-9
    assert np.max(np.abs(pair - exact_pair) / se) > 10.0


def test_strong_logits_known_answer():
    # softmax.rs:873-898: logits [[-10,-10,10,-10], [-10,10,-10,-10]] -> 2, 1
    bias = np.array([[-10, -10, 10, -10], [-10, 10, -10, -10]], np.float32)
    p = orc.Potts(2, 4, np.zeros((0, 2), np.uint32), np.zeros(0, np.float32), bias,
                  [np.array([0, 1], np.uint32)])
    st, _ = p.run_blocks(42, np.zeros((500, 2), np.uint8), 3)
    assert (st[:, p.pos(0)] == 2).all() and (st[:, p.pos(1)] == 1).all()


def test_wide_q_exact_enumeration():
    """q = 20 on a 3-node chain: a site's 20 keystream words span two or
    three ChaCha8 blocks (node 1's words start at word 20 of its block's
    stream, offset 4 in block 1).  Sampled node and pair marginals against
    the exact distribution over all 20^3 states."""
    rng = np.random.default_rng(20)
    q, n = 20, 3
    edges = np.array([(0, 1), (1, 2)], np.uint32)
    W = rng.normal(0, 0.8, (2, q, q)).astype(np.float32)
    bias = rng.normal(0, 0.8, (n, q)).astype(np.float32)
    blocks = [np.array([0, 2], np.uint32), np.array([1], np.uint32)]
    exact_node, exact_pair = _exact_marginals(edges, W, bias, q, n=n)
    p = orc.Potts(n, q, edges, W, bias, blocks)
    C = 20000
    node, pair = _sampled_marginals(p, edges, q, C=C, sweeps=12, key=21, n=n)
    se_node = np.sqrt(exact_node * (1 - exact_node) / C) + 1e-9
    se_pair = np.sqrt(exact_pair * (1 - exact_pair) / C) + 1e-9
    assert np.max(np.abs(node - exact_node) / se_node) < 5.0
    assert np.max(np.abs(pair - exact_pair) / se_pair) < 5.5


def test_wide_q_strong_logits_known_answer():
    # the reference's strong-logit test at q = 40: logit +30 at one category,
    # -30 elsewhere, so the draw is that category (words 0..39 and 40..79 of
    # the block's stream: three ChaCha8 blocks, the second shared)
    q = 40
    bias = np.full((2, q), -30.0, np.float32)
    bias[0, 37] = 30.0
    bias[1, 21] = 30.0
    p = orc.Potts(2, q, np.zeros((0, 2), np.uint32), np.zeros(0, np.float32), bias,
                  [np.array([0, 1], np.uint32)])
    st, _ = p.run_blocks(42, np.zeros((300, 2), np.uint8), 2)
    assert (st[:, p.pos(0)] == 37).all() and (st[:, p.pos(1)] == 21).all()


@pytest.mark.parametrize("q", [300, 1000])
def test_more_than_256_categories_strong_logits(q):
    """States of two bytes per node: logit +30 at a category above 255, -30
    elsewhere, so every draw is that category."""
    bias = np.full((2, q), -30.0, np.float32)
    bias[0, q - 3] = 30.0
    bias[1, 257] = 30.0
    p = orc.Potts(2, q, np.zeros((0, 2), np.uint32), np.zeros(0, np.float32), bias,
                  [np.array([0, 1], np.uint32)])
    st, _ = p.run_blocks(42, np.zeros((50, 2), np.uint16), 2)
    assert st.dtype == np.uint16
    assert (st[:, p.pos(0)] == q - 3).all() and (st[:, p.pos(1)] == 257).all()


def test_more_than_256_categories_exact_enumeration():
    """q = 300 on a 2-node edge: sampled node marginals against the exact
    distribution over all 300^2 states."""
    rng = np.random.default_rng(300)
    q, n = 300, 2
    edges = np.array([(0, 1)], np.uint32)
    W = rng.normal(0, 1.0, (1, q, q)).astype(np.float32)
    bias = rng.normal(0, 1.0, (n, q)).astype(np.float32)
    blocks = [np.array([0], np.uint32), np.array([1], np.uint32)]
    exact_node, _ = _exact_marginals(edges, W, bias, q, n=n)
    p = orc.Potts(n, q, edges, W, bias, blocks)
    C = 8000
    st, _ = p.run_blocks(31, np.zeros((C, p.n_total), np.uint16), 6)
    node = np.stack([np.bincount(st[:, p.pos(k)], minlength=q) / C for k in range(n)])
    se_node = np.sqrt(exact_node * (1 - exact_node) / C) + 1e-9
    assert np.max(np.abs(node - exact_node) / se_node) < 5.5


def test_errors():
    for q in (1, 65537):
        with pytest.raises(ValueError, match="q must lie"):
            orc.Potts(2, q, np.zeros((0, 2), np.uint32), np.zeros(0, np.float32),
                      np.zeros((2, q), np.float32), [np.array([0, 1], np.uint32)])
    bias = np.zeros((3, 2), np.float32)
    with pytest.raises(ValueError, match="empty block"):
        orc.Potts(3, 2, np.zeros((0, 2), np.uint32), np.zeros(0, np.float32), bias,
                  [np.array([0, 1, 2], np.uint32), np.array([], np.uint32)])
    with pytest.raises(ValueError, match="global location map"):
        orc.Potts(3, 2, np.array([[0, 2]], np.uint32), np.zeros(4, np.float32), bias,
                  [np.array([0, 1], np.uint32)])


def _random_potts(n, m, q, seed):
    rng = np.random.default_rng(seed)
    edges = set()
    while len(edges) < m:
        a, b = (int(v) for v in rng.integers(0, n, 2))
        if a != b:
            edges.add((a, b))
    edges = np.array(sorted(edges), np.uint32)
    W = rng.normal(0, 0.8, (len(edges), q, q)).astype(np.float32)
    bias = rng.normal(0, 0.5, (n, q)).astype(np.float32)
    return rng, edges, W, bias


def test_clamped_blocks_theta_identity_and_fixed_values():
    """Clamped blocks (global state = free ++ clamped, blockspec.rs:15-67):
    theta of every free node still satisfies the energy-difference identity
    with the clamped neighbours' values in the energy, the clamped positions
    keep their values through run_blocks, and only free nodes move."""
    rng, edges, W, bias = _random_potts(26, 70, 4, 21)
    n, q = 26, 4
    perm = rng.permutation(n)
    free, clamped = [perm[:9], perm[9:17]], [perm[17:22], perm[22:]]
    p = orc.Potts(n, q, edges, W, bias, free, clamped)
    assert p.n_total == n
    eu, ev = edges[:, 0], edges[:, 1]
    x = rng.integers(0, q, n)
    glob = np.zeros(n, np.uint8)
    for node in range(n):
        glob[p.pos(node)] = x[node]
    th = p.theta(glob)
    for node in np.concatenate(free):
        e = []
        for c in range(q):
            y = x.copy()
            y[node] = c
            e.append(_energy(y, bias, eu, ev, W))
        e = np.array(e)
        assert np.allclose(th[p.pos(node)] - th[p.pos(node), 0], -(e - e[0]), atol=2e-5)
    init = rng.integers(0, q, (6, n)).astype(np.uint8)
    out, _ = p.run_blocks(4, init, 12)
    nf = sum(len(b) for b in free)
    assert np.array_equal(out[:, nf:], init[:, nf:])
    assert not np.array_equal(out[:, :nf], init[:, :nf])


def test_sample_states_follows_the_key_tree_of_run_blocks():
    """orc_potts_sample_states against orc_potts_run_blocks on the key tree of
    sample_with_observation (sampling.rs:178-320): per chain c with key k_c =
    split(key, C)[c], (wk, sk) = k_c.split_two(); observation 0 is the state
    after n_warmup sweeps keyed by wk, observation i + 1 the state after
    steps_per_sample more sweeps keyed by sk.split(n_samples - 1)[i].  A
    one-chain run_blocks takes its key as the chain key (split(key, 1)[0] =
    key)."""
    rng, edges, W, bias = _random_potts(20, 50, 3, 22)
    perm = rng.permutation(20)
    p = orc.Potts(20, 3, edges, W, bias, [perm[:7], perm[7:13], perm[13:]])
    C, sched = 5, (3, 4, 2)
    init = rng.integers(0, 3, (C, 20)).astype(np.uint8)
    out = p.sample_states(77, sched, init)
    assert out.shape == (4, C, 20)
    ck = orc.rng_split(77, C)
    for c in range(C):
        wk, sk = orc.rng_split(ck[c], 2)
        st, _ = p.run_blocks(wk, init[c:c + 1], sched[0])
        assert np.array_equal(out[0, c], st[0])
        for i, k in enumerate(orc.rng_split(sk, sched[1] - 1)):
            st, _ = p.run_blocks(k, st, sched[2])
            assert np.array_equal(out[i + 1, c], st[0])
