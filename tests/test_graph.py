"""Graph builders: crates/thrml-models/src/graph_utils.rs:177-335 and
crates/thrml-examples/src/lib.rs:114-302 (their own tests are the KATs here),
oracle and product implementations side by side."""
import numpy as np
import pytest

import pyoracle as orc
import thrml_hip as th


@pytest.mark.parametrize("impl", ["oracle", "product"])
def test_lattice_edge_counts(impl):
    def edges(side, torus):
        if impl == "oracle":
            return orc.lattice_edges(side, torus)
        return th.make_nearest_neighbor_lattice(side, torus)[1]

    assert edges(4, False).shape[0] == 24  # graph_utils.rs:306-316
    assert edges(4, True).shape[0] == 32   # graph_utils.rs:318-328
    assert edges(6, True).shape[0] == 72
    assert edges(2, True).shape[0] == 4    # 2x2 torus: duplicates removed


def test_odd_side_rounds_up():
    n, e, up, lo = th.make_nearest_neighbor_lattice(5, False)
    assert n == 36  # graph_utils.rs:285-291
    assert len(up) == 18 and len(lo) == 18


def test_zero_side_len_rejected():
    # graph_utils.rs:330-334 (make_lattice_graph(0, ...) panics)
    with pytest.raises(th.ThrmlError, match="side_len must be positive"):
        th.make_nearest_neighbor_lattice(0, False)


def test_blocks_disjoint_and_cover():
    for side in (4, 6, 64):
        n, e, up, lo = th.make_nearest_neighbor_lattice(side, True)
        a, b = set(up.nodes.tolist()), set(lo.nodes.tolist())
        assert not (a & b) and (a | b) == set(range(n))  # graph_utils.rs:293-304
        # checkerboard: every edge joins the two blocks
        col = np.zeros(n, int)
        col[lo.nodes] = 1
        assert np.all(col[e[:, 0]] != col[e[:, 1]])


def test_canonical_order_oracle_equals_product():
    for side, torus in [(4, True), (4, False), (8, True), (64, True), (2, True)]:
        a = orc.lattice_edges(side, torus)
        b = th.make_nearest_neighbor_lattice(side, torus)[1]
        assert np.array_equal(a, b)
        up_o, lo_o = orc.lattice_blocks(side)
        _, _, up, lo = th.make_nearest_neighbor_lattice(side, torus)
        assert np.array_equal(up_o, up.nodes) and np.array_equal(lo_o, lo.nodes)
        # edges are (min, max) and unique
        assert np.all(a[:, 0] < a[:, 1])
        assert len({tuple(x) for x in a.tolist()}) == a.shape[0]


def test_greedy_coloring_chain_and_lattice():
    chain = np.array([[i, i + 1] for i in range(4)])
    c, k = orc.greedy_coloring(5, chain)
    assert k == 2 and np.array_equal(c, th.greedy_coloring(5, chain))  # lib.rs:262-271
    n, e, _, _ = th.make_nearest_neighbor_lattice(8, True)
    c = th.greedy_coloring(n, e)
    assert c.max() + 1 == 2
    assert np.all(c[e[:, 0]] != c[e[:, 1]])


def test_greedy_coloring_random_graph_proper():
    rng = np.random.default_rng(0)
    n = 500
    e = rng.integers(0, n, (3000, 2))
    e = e[e[:, 0] != e[:, 1]]
    c_o, k = orc.greedy_coloring(n, e)
    c_p = th.greedy_coloring(n, e)
    assert np.array_equal(c_o, c_p)
    assert np.all(c_p[e[:, 0]] != c_p[e[:, 1]])
    blocks = th.coloring_to_blocks(c_p)
    assert len(blocks) == k and sum(len(b) for b in blocks) == n
    for i, b in enumerate(blocks):
        assert np.all(c_p[b.nodes] == i) and np.all(np.diff(b.nodes.astype(int)) > 0)


def test_erdos_renyi_properties():
    n, p = 20000, 12.0 / 19999
    e = th.erdos_renyi(n, p, 2003)
    m = e.shape[0]
    mean = p * n * (n - 1) / 2
    assert abs(m - mean) < 5 * np.sqrt(mean)
    assert np.all(e[:, 0] < e[:, 1]) and e.max() < n
    key = e[:, 0].astype(np.int64) * n + e[:, 1]
    assert np.all(np.diff(key) > 0)  # strictly ascending (min, max): no duplicates
    deg = np.bincount(e.ravel(), minlength=n)
    assert abs(deg.mean() - 12.0) < 0.2 and abs(deg.var() - 12.0) < 1.0  # Poisson(12)
    assert np.array_equal(e, th.erdos_renyi(n, p, 2003))


def test_param_normal_oracle_equals_product():
    a = orc.param_normal(1002, 10001, 0.44, 0.05)
    b = th.param_normal(1002, 10001, 0.44, 0.05)
    assert np.array_equal(a, b)
    x = th.param_normal(7, 200_000, 0.0, 1.0).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 1) < 0.01


def test_double_grid_structure():
    """The MNIST model's double grid (test_train_mnist.rs:177-225 asserts the
    counts): 40 x 40 layers, jumps (1, 4, 15), 814 visible nodes."""
    up, lo, vis, rest, n, e = th.double_grid(40, [1, 4, 15], 28 * 28 + 30, 0)
    assert len(up) == 1600 and len(lo) == 1600 and n == 3200
    assert len(vis) == 814 and len(rest) == 1600 - 814
    assert e.shape == (1600 * 13, 2)
    # every edge joins upper i to lower j at torus displacement 0 or (+-d, 0), (0, +-d)
    i, j = e[:, 0].astype(np.int64), e[:, 1].astype(np.int64) - 1600
    assert (i < 1600).all() and (j >= 0).all() and (j < 1600).all()
    assert np.array_equal(i[:1600], np.arange(1600)) and np.array_equal(j[:1600], np.arange(1600))
    dr, dc = (j // 40 - i // 40) % 40, (j % 40 - i % 40) % 40
    for q, d in enumerate([1, 4, 15]):
        s = slice(1600 + 6400 * q, 1600 + 6400 * (q + 1))
        want_r = np.tile([(-d) % 40, d, 0, 0], 1600)
        want_c = np.tile([0, 0, (-d) % 40, d], 1600)
        assert np.array_equal(dr[s], want_r) and np.array_equal(dc[s], want_c)
        assert np.array_equal(i[s], np.repeat(np.arange(1600), 4))
    assert len(set(map(tuple, e.tolist()))) == e.shape[0]  # no repeated edge at these jumps
    v = vis.nodes
    assert len(set(v.tolist())) == 814 and v.max() < 1600
    assert np.array_equal(np.sort(np.concatenate([v, rest.nodes])), np.arange(1600))
    assert np.all(np.diff(rest.nodes.astype(np.int64)) > 0)
    # bipartite: the two-block colourings the training test samples with are proper
    col = np.zeros(n, int)
    col[lo.nodes] = 1
    assert np.all(col[e[:, 0]] != col[e[:, 1]])
    with pytest.raises(th.ThrmlError):
        th.double_grid(4, [1], 17, 0)


def test_double_grid_visible_shuffle_uniform():
    """The visible nodes are a prefix of a Fisher-Yates shuffle (rand 0.8.5
    SliceRandom::shuffle on StdRng): over seeds, all 24 orders of a 2 x 2 grid
    appear about equally often.  A draw from 0..i instead of 0..=i (Sattolo's
    cycles) would reach 6 of them; the exact word stream of the ChaCha12
    generator is not pinned by any vector the reference holds."""
    counts = {}
    for seed in range(2400):
        p = tuple(th.double_grid(2, [], 3, seed)[2].nodes.tolist())  # 3 fix the order
        counts[p] = counts.get(p, 0) + 1
    assert len(counts) == 24
    c = np.array(list(counts.values()), float)
    chi2 = ((c - 100.0) ** 2 / 100.0).sum()
    assert chi2 < 60.0  # 23 degrees of freedom: p about 4e-5
    assert not np.array_equal(th.double_grid(40, [1], 814, 0)[2].nodes,
                              th.double_grid(40, [1], 814, 1)[2].nodes)
