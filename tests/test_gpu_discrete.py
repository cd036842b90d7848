"""Programs over general discrete factors on the device (FactorSamplingProgram,
crates/thrml-models/src/factor.rs:126-185; DiscreteEBMFactor,
crates/thrml-models/src/discrete_ebm.rs:293-593; SpinGibbsConditional and
CategoricalGibbsConditional, crates/thrml-samplers/src/spin_gibbs.rs:512-595,
softmax.rs:586-710) against the oracle, bit for bit:

  - mixed models with higher-order spin factors, spin-categorical and
    categorical-categorical factors, spin and categorical blocks; run_blocks,
    sample_states and energies; 5 to 130 chains; q = 2, 3, 7, 8, 10, 16, 20, 48,
    and 257, 300, 1000 (two bytes of state per node);
  - clamped blocks, superblocks, and blocks whose nodes interact (staged);
  - a spin head of a factor with two categorical groups (first tail only);
  - square factors (SquareDiscreteEBMFactor / SquareCategoricalEBMFactor,
    discrete_ebm.rs:858-1064): the merged categorical-head group, nodes in
    both roles, with and without spin tails;
  - an IsingEBM and Potts models (q = 2, 3, 5, 6, 19, 24, 26, 48, 300) written as factors equal
    the Ising (CSR kernel) and categorical programs on the same inputs;
  - the constructor's checks."""
import numpy as np
import pytest

import pyoracle as orc
import thrml_hip as th
from conftest import log_case

pytestmark = pytest.mark.gpu


def _mixed(rng, n_spin, n_cat, q, m):
    S = np.arange(n_spin)
    X = np.arange(n_spin, n_spin + n_cat)

    def pick(pool, k):
        rows = [rng.choice(pool, k, replace=False) for _ in range(m)]
        return [np.array([r[i] for r in rows], np.uint32) for i in range(k)]

    f = [([S], [], rng.normal(0, 0.5, (n_spin, 1, 1))),
         (pick(S, 2), [], rng.normal(0, 0.6, (m, 1, 1))),
         (pick(S, 3), [], rng.normal(0, 0.6, (m, 1, 1))),
         (pick(S, 1), pick(X, 1), rng.normal(0, 0.6, (m, q, 1))),
         ([], [X], rng.normal(0, 0.5, (n_cat, q, 1))),
         ([], pick(X, 2), rng.normal(0, 0.6, (m, q, q))),
         (pick(S, 2), pick(X, 1), rng.normal(0, 0.6, (m, q, 1))),
         (pick(S, 1), pick(X, 2), rng.normal(0, 0.6, (m, q, q)))]
    return [(sg, cg, np.asarray(w, np.float32)) for sg, cg, w in f]


def _programs(device, n, kinds, q, factors, free, clamped=(), superblocks=None):
    fs = [(th.SquareDiscreteEBMFactor if f[3:] and f[3] else th.DiscreteEBMFactor)(*f[:3])
          for f in factors]
    nested = free if superblocks is None else [
        [free[b] for b in range(superblocks[s], superblocks[s + 1])]
        for s in range(len(superblocks) - 1)]
    prog = th.FactorSamplingProgram(kinds, q, fs, nested, clamped, device)
    o = orc.Discrete(n, kinds, q, factors, free, clamped, superblocks=superblocks)
    return prog, o


def _init(rng, kinds, q, C, blocks):
    """Random states in global position order (the blocks' concatenation)."""
    kp = kinds[np.concatenate([np.asarray(b) for b in blocks])]
    return np.where(kp[None, :] == 0, rng.integers(0, 2, (C, kp.size)),
                    rng.integers(0, q, (C, kp.size))).astype(np.uint8 if q <= 256 else np.uint16)


def _parity(prog, o, init, key, n_iters):
    C = init.shape[0]
    st = prog.new_state(C)
    st.set_global(init)
    th.run_blocks(th.RngKey(key), prog, st, (), n_iters)
    got = st.get_global()
    want, _ = o.run_blocks(key, init, n_iters)
    assert np.array_equal(got, want)
    e = th.discrete_energy(prog, st)
    ew = o.energy(want)
    assert np.abs(e - ew).max() <= 1e-9 * max(1.0, np.abs(ew).max())
    st.set_global(init)
    samples = th.sample_states(th.RngKey(key + 1), prog, th.SamplingSchedule(2, 4, 2), st)
    assert np.array_equal(samples, o.sample_states(key + 1, (2, 4, 2), init))
    st.close()


@pytest.mark.parametrize("q,C", [(3, 5), (8, 70), (16, 130), (2, 33), (7, 64), (10, 32),
                                 (20, 40), (48, 9)])
def test_mixed_higher_order_model(device, q, C):
    rng = np.random.default_rng(q)
    n_spin, n_cat = 300, 200
    n = n_spin + n_cat
    kinds = np.r_[np.zeros(n_spin), np.ones(n_cat)].astype(np.uint8)
    factors = _mixed(rng, n_spin, n_cat, q, 400)
    # one node per block would be exact Gibbs; random blocks test the slot
    # machinery (nodes of a block interact: every block is staged)
    perm_s, perm_c = rng.permutation(n_spin), n_spin + rng.permutation(n_cat)
    free = [perm_s[:150], perm_c[:100], perm_s[150:], perm_c[100:]]
    log_case(f"discrete mixed model q={q} C={C}")
    prog, o = _programs(device, n, kinds, q, factors, free)
    assert prog.kind == "discrete"
    _parity(prog, o, _init(rng, kinds, q, C, free), 17, 4)


@pytest.mark.parametrize("q,C,m", [(300, 9, 40), (1000, 4, 8), (257, 64, 40)])
def test_more_than_256_categories_mixed_model(device, q, C, m):
    """Categorical nodes with more than 256 categories (two bytes of state per
    node): the spin blocks read two-byte tails, the categorical blocks run
    the wide kernel on two-byte states; sweeps, sample_states (returned as
    uint16) and energies equal the oracle's."""
    rng = np.random.default_rng(q + C)
    n_spin, n_cat = 60, 40
    n = n_spin + n_cat
    kinds = np.r_[np.zeros(n_spin), np.ones(n_cat)].astype(np.uint8)
    factors = _mixed(rng, n_spin, n_cat, q, m)
    perm_s, perm_c = rng.permutation(n_spin), n_spin + rng.permutation(n_cat)
    free = [perm_s[:30], perm_c[:20], perm_s[30:], perm_c[20:]]
    log_case(f"discrete mixed model q={q} C={C}")
    prog, o = _programs(device, n, kinds, q, factors, free)
    init = _init(rng, kinds, q, C, free)
    assert init.max() > 255
    _parity(prog, o, init, 19, 3)


def test_wave_and_lane_factor_kernels_either_side_of_the_choice(device):
    """q = 300 categorical blocks of 4096 sites on either side of the wave /
    lane kernel choice (16 chains: 65,536 items per block on the wave kernel;
    20 chains: 81,920 on the lane kernel), with spin nodes coupled to some of
    them (two-byte spin tails), each against the oracle."""
    q, n_spin, n_cat = 300, 64, 8192
    n = n_spin + n_cat
    rng = np.random.default_rng(3)
    kinds = np.r_[np.zeros(n_spin), np.ones(n_cat)].astype(np.uint8)
    S, X = np.arange(n_spin, dtype=np.uint32), np.arange(n_spin, n, dtype=np.uint32)
    factors = [([S], [], rng.normal(0, 0.5, (n_spin, 1, 1)).astype(np.float32)),
               ([], [X], rng.normal(0, 1.0, (n_cat, q, 1)).astype(np.float32)),
               ([S], [X[:n_spin]], rng.normal(0, 0.8, (n_spin, q, 1)).astype(np.float32))]
    free = [S, X[0::2], X[1::2]]
    prog, o = _programs(device, n, kinds, q, factors, free)
    for C in (16, 20):
        log_case(f"discrete q=300 wave/lane choice C={C}")
        init = _init(rng, kinds, q, C, free)
        st = prog.new_state(C)
        st.set_global(init)
        th.run_blocks(th.RngKey(C), prog, st, (), 2)
        want, _ = o.run_blocks(C, init, 2)
        assert np.array_equal(st.get_global(), want)
        st.close()


@pytest.mark.parametrize("q,m", [(5, 150), (300, 30)])
def test_clamped_blocks_and_superblocks(device, q, m):
    rng = np.random.default_rng(31)
    n_spin, n_cat = 120, 80
    n = n_spin + n_cat
    kinds = np.r_[np.zeros(n_spin), np.ones(n_cat)].astype(np.uint8)
    factors = _mixed(rng, n_spin, n_cat, q, m)
    free = [np.arange(0, 60), np.arange(120, 160), np.arange(60, 100), np.arange(160, 190)]
    clamped = [np.arange(100, 120), np.arange(190, 200)]
    log_case(f"discrete clamped blocks + superblocks [0, 2, 4], q={q}")
    prog, o = _programs(device, n, kinds, q, factors, free, clamped, superblocks=[0, 2, 4])
    init = _init(rng, kinds, q, 37, free + clamped)
    _parity(prog, o, init, 23, 3)
    st = prog.new_state(37)
    st.set_global(init)
    th.run_blocks(th.RngKey(5), prog, st, (), 3)
    nf = sum(len(b) for b in free)
    assert np.array_equal(st.get_global()[:, nf:], init[:, nf:])
    st.close()


def test_spin_head_with_two_categorical_tails(device):
    rng = np.random.default_rng(41)
    q, m = 4, 64
    S = np.arange(m)
    X, Y = np.arange(m, 2 * m), np.arange(2 * m, 3 * m)
    kinds = np.r_[np.zeros(m), np.ones(2 * m)].astype(np.uint8)
    factors = [([S], [X, Y], rng.normal(0, 1.0, (m, q, q)).astype(np.float32)),
               ([S], [], rng.normal(0, 0.5, (m, 1, 1)).astype(np.float32))]
    free = [S, X, Y]
    log_case("discrete spin head with two categorical tails")
    prog, o = _programs(device, 3 * m, kinds, q, factors, free)
    _parity(prog, o, _init(rng, kinds, q, 33, free), 29, 5)


@pytest.mark.parametrize("q,C,with_spins", [(4, 45, False), (6, 64, True), (16, 9, True)])
def test_square_factors(device, q, C, with_spins):
    rng = np.random.default_rng(71 + q)
    n_spin, n_cat, m = (80 if with_spins else 0), 150, 500
    n = n_spin + n_cat
    kinds = np.r_[np.zeros(n_spin), np.ones(n_cat)].astype(np.uint8)
    S, X = np.arange(n_spin), np.arange(n_spin, n)
    rows = [rng.choice(X, 2, replace=False) for _ in range(m)]
    U = np.array([r[0] for r in rows], np.uint32)
    V = np.array([r[1] for r in rows], np.uint32)
    sg = [rng.choice(S, m).astype(np.uint32)] if with_spins else []
    factors = [(sg, [U, V], rng.normal(0, 0.7, (m, q, q)).astype(np.float32), True),
               ([], [X], rng.normal(0, 0.5, (n_cat, q, 1)).astype(np.float32))]
    if with_spins:
        factors.append(([S], [], rng.normal(0, 0.5, (n_spin, 1, 1)).astype(np.float32), True))
    free = ([S[::2], S[1::2]] if with_spins else []) + [X[::3], X[1::3], X[2::3]]
    log_case(f"discrete square factors q={q} C={C} spins={with_spins}")
    prog, o = _programs(device, n, kinds, q, factors, free)
    _parity(prog, o, _init(rng, kinds, q, C, free), 37, 4)
    # SquareCategoricalEBMFactor is the categorical-only square factor
    cat = th.FactorSamplingProgram(kinds, q, [th.SquareCategoricalEBMFactor([U, V], factors[0][2])]
                                   + [th.DiscreteEBMFactor(*f[:3]) for f in factors[1:]], free, [],
                                   device) if not with_spins else None
    if cat is not None:
        init = _init(rng, kinds, q, C, free)
        a, b = prog.new_state(C), cat.new_state(C)
        a.set_global(init)
        b.set_global(init)
        th.run_blocks(th.RngKey(2), prog, a, (), 3)
        th.run_blocks(th.RngKey(2), cat, b, (), 3)
        assert np.array_equal(a.get_global(), b.get_global())
        a.close()
        b.close()


@pytest.mark.parametrize("q,C", [(8, 32), (4, 33), (3, 64)])
def test_nodes_without_factors(device, q, C):
    """Spin and categorical nodes that no factor touches, last in their
    blocks and last in the position order: their sites have no slots (the
    interleaved sums read past them and add nothing); a few weights only."""
    rng = np.random.default_rng(90 + q)
    ns, nc = 12, 12
    n = ns + nc
    kinds = np.r_[np.zeros(ns), np.ones(nc)].astype(np.uint8)
    factors = [([np.array([0, 2, 4], np.uint32), np.array([1, 3, 5], np.uint32)], [],
                 rng.normal(0, 0.6, (3, 1, 1)).astype(np.float32)),
               ([], [np.array([12, 14], np.uint32)], rng.normal(0, 0.6, (2, q, 1)).astype(np.float32))]
    free = [np.arange(0, 12, 2), np.arange(1, 12, 2), np.arange(12, 24, 2), np.arange(13, 24, 2)]
    log_case(f"discrete nodes without factors q={q} C={C}")
    prog, o = _programs(device, n, kinds, q, factors, free)
    _parity(prog, o, _init(rng, kinds, q, C, free), 71, 3)


@pytest.mark.parametrize("C", [7, 100])
def test_ising_as_factors_equals_ising_program(device, C):
    n = 400
    rng = np.random.default_rng(51)
    e = set()
    while len(e) < 1200:
        a, b = (int(v) for v in rng.integers(0, n, 2))
        if a != b:
            e.add((a, b))
    edges = np.array(sorted(e), np.uint32)
    b = rng.normal(0, 0.4, n).astype(np.float32)
    J = rng.normal(0, 0.5, len(edges)).astype(np.float32)
    beta = np.float32(0.8)
    col, _ = orc.greedy_coloring(n, edges)
    blocks = [np.nonzero(col == c)[0].astype(np.uint32) for c in range(int(col.max()) + 1)]
    ising = th.IsingSamplingProgram(th.IsingEBM(n, edges, b, J, beta), blocks, [], device)
    assert ising.kind == "csr"
    fs = [th.SpinEBMFactor([np.arange(n)], (beta * b).reshape(n, 1, 1)),
          th.SpinEBMFactor([edges[:, 0], edges[:, 1]], (beta * J).reshape(-1, 1, 1))]
    disc = th.FactorSamplingProgram(np.zeros(n, np.uint8), 0, fs, blocks, [], device)
    init = rng.integers(0, 2, (C, n)).astype(np.uint8)
    log_case(f"Ising as factors vs IsingSamplingProgram, C={C}")
    a, d = ising.new_state(C), disc.new_state(C)
    a.set_global(init)
    d.set_global(init)
    th.run_blocks(th.RngKey(3), ising, a, (), 6)
    th.run_blocks(th.RngKey(3), disc, d, (), 6)
    assert np.array_equal(a.get_global(), d.get_global())
    a.close()
    d.close()


@pytest.mark.parametrize("q,n,m,C", [(6, 300, 800, 40), (5, 2000, 6000, 64), (3, 1000, 3000, 33),
                                     (2, 700, 2000, 65), (24, 300, 800, 33), (48, 200, 500, 17),
                                     (26, 150, 400, 9), (19, 150, 400, 6), (300, 100, 200, 9)])
def test_potts_as_factors_equals_categorical_program(device, q, n, m, C):
    # q = 2, 3, 5, 6: runs of 8 or 16 sites split into 4-site parts in both
    # kernels; q = 19, 24, 26, 48: the two wide kernels (each row load form)
    rng = np.random.default_rng(61 + q)
    e = set()
    while len(e) < m:
        a, b = (int(v) for v in rng.integers(0, n, 2))
        if a != b:
            e.add((a, b))
    edges = np.array(sorted(e), np.uint32)
    W = rng.normal(0, 0.6, (len(edges), q, q)).astype(np.float32)
    bias = rng.normal(0, 0.5, (n, q)).astype(np.float32)
    col, _ = orc.greedy_coloring(n, edges)
    blocks = [np.nonzero(col == c)[0].astype(np.uint32) for c in range(int(col.max()) + 1)]
    potts = th.CategoricalProgram(n, q, edges, W, bias, blocks, device)
    fs = [th.CategoricalEBMFactor([np.arange(n)], bias.reshape(n, q, 1)),
          th.CategoricalEBMFactor([edges[:, 0], edges[:, 1]], W)]
    disc = th.FactorSamplingProgram(np.ones(n, np.uint8), q, fs, blocks, [], device)
    init = rng.integers(0, q, (C, n)).astype(np.uint8 if q <= 256 else np.uint16)
    log_case(f"Potts as factors vs CategoricalProgram q={q} n={n} C={C}")
    a, d = potts.new_state(C), disc.new_state(C)
    a.set_global(init)
    d.set_global(init)
    th.run_blocks(th.RngKey(8), potts, a, (), 5)
    th.run_blocks(th.RngKey(8), disc, d, (), 5)
    assert np.array_equal(a.get_global(), d.get_global())
    ea, ed = th.potts_energy(potts, a), th.discrete_energy(disc, d)
    assert np.abs(ea - ed).max() <= 1e-9 * np.abs(ea).max()
    a.close()
    d.close()


def test_constructor_checks_and_state_values(device):
    kinds = np.array([0, 0, 1, 1], np.uint8)
    blocks = [np.array([0, 1]), np.array([2, 3])]
    cases = [
        ([th.DiscreteEBMFactor([[0]], [], np.zeros((1, 2, 1)))], "weights \\[b, 1, 1\\]"),
        ([th.DiscreteEBMFactor([[2]], [], np.zeros((1, 1, 1)))], "spin node groups must hold"),
        ([th.DiscreteEBMFactor([], [[2]], np.zeros((1, 2, 1)))], "weights \\[b, q, 1\\]"),
        ([th.DiscreteEBMFactor([], [[2], [3]], np.zeros((1, 3, 2)))], "weights \\[b, q, q\\]"),
        ([th.DiscreteEBMFactor([], [[2]], np.zeros((1, 1, 1)))], "effective dims"),
    ]
    for fs, msg in cases:
        with pytest.raises(th.ThrmlError, match=msg):
            th.FactorSamplingProgram(kinds, 3, fs, blocks, [], device)
    for w in (np.zeros((1, 3, 2)), np.zeros((1, 3, 1))):
        with pytest.raises(th.ThrmlError, match="Interaction tensor is not square"):
            th.SquareDiscreteEBMFactor([], [[2], [3]], w)
    # the library's own check, past the host-side one
    f = th.DiscreteEBMFactor([], [[2], [3]], np.zeros((1, 3, 2)))
    f.flags = 1
    with pytest.raises(th.ThrmlError, match="Interaction tensor is not square"):
        th.FactorSamplingProgram(kinds, 3, [f], blocks, [], device)
    with pytest.raises(th.ThrmlError, match="both spin and categorical"):
        th.FactorSamplingProgram(kinds, 3, [], [np.array([1, 2])], [], device)
    prog = th.FactorSamplingProgram(kinds, 3, [th.DiscreteEBMFactor([[0]], [[2]], np.ones((1, 3, 1)))],
                                    blocks, [], device)
    st = prog.new_state(2)
    with pytest.raises(th.ThrmlError, match="spin value out of range"):
        st.set_block(0, np.array([[0, 2], [1, 1]], np.uint8))
    with pytest.raises(th.ThrmlError, match="category value out of range"):
        st.set_block(1, np.array([[0, 3], [1, 1]], np.uint8))
    st.set_block(1, np.array([[0, 2], [1, 1]], np.uint8))
    assert np.array_equal(st.get_block(1), [[0, 2], [1, 1]])
    st.close()
