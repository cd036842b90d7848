"""Pins of the oracle's general discrete-factor program (orc_discrete.c:
DiscreteEBMFactor, crates/thrml-models/src/discrete_ebm.rs:293-593, sampled by
SpinGibbsConditional / CategoricalGibbsConditional, crates/thrml-samplers/src/
spin_gibbs.rs:512-595, softmax.rs:586-710) that do not retype its formulas.

  - reductions: an IsingEBM written as SpinEBMFactor([all], beta b) +
    SpinEBMFactor([U, V], beta J) (ising.rs:105-143) samples bit for bit as the
    separately written Ising oracle, with clamped blocks and superblocks; a
    Potts model written as CategoricalEBMFactor bias + edge factors samples
    as the Potts oracle (discrete_ebm.rs:456-548; q = 3, 5, 24, 40);
  - the energy-difference identity on mixed and higher-order models: gamma of a
    spin = -(E(s=1) - E(s=0)) / 2 and theta[c] - theta[0] = -(E(c) - E(0)),
    with E evaluated from the raw factors (factor_energy), not from the slots
    (q = 4, 20);
  - exact enumeration: a 3-spin + 2-categorical model with a three-body spin
    factor, spin-categorical and categorical-categorical factors; sampled
    marginals within 5 standard errors of the exact Boltzmann marginals, and a
    planted mistake (either sign of a spin product, or the swapped axis of the
    second categorical head) moves them by more than 10;
  - the rule SpinGibbsConditional applies to a factor with two categorical
    groups: the weight row flattened to q*q entries, indexed by the first
    categorical tail only (spin_gibbs.rs:553-575);
  - the constructor's checks (discrete_ebm.rs:300-358);
  - SquareDiscreteEBMFactor (discrete_ebm.rs:858-1013), whose two
    categorical-head groups are merged into one accumulation (u-role rows,
    then v-role rows): its theta equals bit for bit that of the unmerged
    factor [U ++ V, V' ++ U'], [W; W^T], whose tails V', U' are clamped
    shadow copies of V, U (its first head group is then the merged group, and
    its second heads only the shadows), and differs from the unmerged
    [U, V], W in rounding at some position; spin heads and the energies are
    unchanged; "Interaction tensor is not square"."""
import itertools

import numpy as np
import pytest

import pyoracle as orc


def _graph(n, m, seed):
    rng = np.random.default_rng(seed)
    e = set()
    while len(e) < m:
        a, b = (int(v) for v in rng.integers(0, n, 2))
        if a != b:
            e.add((a, b))
    return rng, np.array(sorted(e), np.uint32)


def _colour_blocks(n, edges):
    col, _ = orc.greedy_coloring(n, edges)
    return [np.nonzero(col == c)[0].astype(np.uint32) for c in range(int(col.max()) + 1)]


@pytest.mark.parametrize("clamp,superblocks", [(False, None), (True, None), (False, "pair")])
def test_ising_written_as_factors_equals_ising_oracle(clamp, superblocks):
    n = 120
    rng, edges = _graph(n, 300, 1)
    b = rng.normal(0, 0.5, n).astype(np.float32)
    J = rng.normal(0, 0.6, len(edges)).astype(np.float32)
    beta = np.float32(0.9)
    blocks = _colour_blocks(n, edges)
    free, clamped = (blocks[:-1], blocks[-1:]) if clamp else (blocks, [])
    sb = None if superblocks is None else [0, 2] + list(range(3, len(free) + 1))
    ising = orc.Ising(n, edges, b, J, beta, free, clamped, superblocks=sb)
    factors = [([np.arange(n)], [], (beta * b).reshape(n, 1, 1)),
               ([edges[:, 0], edges[:, 1]], [], (beta * J).reshape(-1, 1, 1))]
    disc = orc.Discrete(n, np.zeros(n, np.uint8), 0, factors, free, clamped, superblocks=sb)
    C = 9
    init = rng.integers(0, 2, (C, n)).astype(np.uint8)
    a, _ = ising.run_blocks(44, init, 5)
    d, _ = disc.run_blocks(44, init, 5)
    assert np.array_equal(a, d)
    assert np.array_equal(ising.sample_states(45, (2, 4, 3), init),
                          disc.sample_states(45, (2, 4, 3), init))
    nf = sum(x.size for x in free)
    assert np.array_equal(ising.gamma(init[0])[:nf], disc.params(init[0])[:, 0])
    # -beta (sum b s + sum J s s) in double against the sum of fl(beta w) terms
    assert np.allclose(ising.energy(init), disc.energy(init), rtol=0, atol=1e-6 * (
        np.abs(beta * b).sum() + np.abs(beta * J).sum()))


@pytest.mark.parametrize("q,clamp", [(3, False), (5, True), (24, False), (40, True), (300, True)])
def test_potts_written_as_factors_equals_potts_oracle(q, clamp):
    n = 90
    rng, edges = _graph(n, 200, 2 + q)
    W = rng.normal(0, 0.6, (len(edges), q, q)).astype(np.float32)
    bias = rng.normal(0, 0.5, (n, q)).astype(np.float32)
    blocks = _colour_blocks(n, edges)
    free, clamped = (blocks[:-1], blocks[-1:]) if clamp else (blocks, [])
    potts = orc.Potts(n, q, edges, W, bias, free, clamped)
    factors = [([], [np.arange(n)], bias.reshape(n, q, 1)),
               ([], [edges[:, 0], edges[:, 1]], W)]
    disc = orc.Discrete(n, np.ones(n, np.uint8), q, factors, free, clamped)
    C = 7
    init = rng.integers(0, q, (C, n)).astype(np.uint16)
    a, _ = potts.run_blocks(61, init, 4)
    d, _ = disc.run_blocks(61, init, 4)
    assert np.array_equal(a, d)
    nf = sum(x.size for x in free)
    assert np.array_equal(potts.theta(init[0])[:nf], disc.params(init[0]))
    assert np.allclose(potts.energy(init), disc.energy(init), rtol=0, atol=1e-9 * (
        np.abs(W).sum() + np.abs(bias).sum()))


def _mixed_model(rng, n_spin, n_cat, q, m):
    """Random factors over spins 0..n_spin-1 and categorical nodes after them:
    spin biases, 2- and 3-body spin factors, spin-categorical factors,
    categorical biases and categorical pair factors (no factor with a spin
    head and two categorical groups)."""
    S = np.arange(n_spin)
    X = np.arange(n_spin, n_spin + n_cat)

    def pick(pool, k):
        rows = [rng.choice(pool, k, replace=False) for _ in range(m)]
        return [np.array([r[i] for r in rows], np.uint32) for i in range(k)]

    f = [([S], [], rng.normal(0, 0.5, (n_spin, 1, 1)))]
    f.append((pick(S, 2), [], rng.normal(0, 0.6, (m, 1, 1))))
    f.append((pick(S, 3), [], rng.normal(0, 0.6, (m, 1, 1))))
    sx = [pick(S, 1)[0], pick(X, 1)[0]]
    f.append(([sx[0]], [sx[1]], rng.normal(0, 0.6, (m, q, 1))))
    sxx = pick(S, 1) + pick(X, 1)
    f.append(([sxx[0]], [sxx[1]], rng.normal(0, 0.6, (m, q, 1))))
    f.append(([], [X], rng.normal(0, 0.5, (n_cat, q, 1))))
    f.append(([], pick(X, 2), rng.normal(0, 0.6, (m, q, q))))
    f.append((pick(S, 2), pick(X, 1), rng.normal(0, 0.6, (m, q, 1))))
    return [(sg, cg, np.asarray(w, np.float32)) for sg, cg, w in f]


@pytest.mark.parametrize("q", [4, 20, 300])
def test_energy_difference_identity_mixed_higher_order(q):
    rng = np.random.default_rng(7 + q)
    n_spin, n_cat = 12, 8
    n = n_spin + n_cat
    kinds = np.r_[np.zeros(n_spin), np.ones(n_cat)].astype(np.uint8)
    factors = _mixed_model(rng, n_spin, n_cat, q, 15)
    free = [np.arange(0, 6), np.arange(6, 12), np.arange(12, 16), np.arange(16, 20)]
    p = orc.Discrete(n, kinds, q, factors, free)
    scale = sum(np.abs(w).sum() for _, _, w in factors)
    for t in range(20):
        st = np.r_[rng.integers(0, 2, n_spin), rng.integers(0, q, n_cat)].astype(np.uint16)
        par = p.params(st)
        for k in range(n):
            node = k  # free blocks list the nodes in order
            if k < n_spin:
                up, dn = st.copy(), st.copy()
                up[node], dn[node] = 1, 0
                e = p.energy(np.stack([up, dn]))
                assert abs(par[k, 0] - (-(e[0] - e[1]) / 2)) < 1e-5 * scale
            else:
                sts = np.repeat(st[None], q, 0)
                sts[:, node] = np.arange(q)
                e = p.energy(sts)
                want = -(e - e[0])
                got = par[k] - par[k, 0]
                assert np.abs(got - want).max() < 1e-5 * scale


def _exact_marginals(n_spin, n_cat, q, factors, energy_fn):
    states = np.array([list(s) + list(x) for s in itertools.product([0, 1], repeat=n_spin)
                       for x in itertools.product(range(q), repeat=n_cat)], np.uint8)
    e = energy_fn(states)
    w = np.exp(-(e - e.min()))
    w /= w.sum()
    ps = np.array([(w * (states[:, i] == 1)).sum() for i in range(n_spin)])
    pc = np.array([[(w * (states[:, n_spin + j] == c)).sum() for c in range(q)]
                   for j in range(n_cat)])
    return ps, pc


def _sampled_marginals(p, n_spin, n_cat, q, C, sweeps, seed):
    rng = np.random.default_rng(seed)
    init = np.c_[rng.integers(0, 2, (C, n_spin)), rng.integers(0, q, (C, n_cat))].astype(np.uint8)
    st, _ = p.run_blocks(seed, init, sweeps)
    ps = (st[:, :n_spin] == 1).mean(0)
    pc = np.array([[(st[:, n_spin + j] == c).mean() for c in range(q)] for j in range(n_cat)])
    return ps, pc


def _tiny():
    rng = np.random.default_rng(11)
    q = 3
    f = [([np.array([0, 1, 2])], [], rng.normal(0, 0.4, (3, 1, 1))),
         ([np.array([0]), np.array([1]), np.array([2])], [], np.array([[[0.9]]])),
         ([np.array([0, 2])], [np.array([3, 4])], rng.normal(0, 0.8, (2, q, 1))),
         ([], [np.array([3, 4])], rng.normal(0, 0.5, (2, q, 1))),
         ([], [np.array([3]), np.array([4])], rng.normal(0, 0.9, (1, q, q))),
         ([np.array([1])], [np.array([3])], rng.normal(0, 0.7, (1, q, 1)))]
    return q, [(sg, cg, np.asarray(w, np.float32)) for sg, cg, w in f]


def test_exact_enumeration_of_a_mixed_model():
    q, factors = _tiny()
    kinds = np.array([0, 0, 0, 1, 1], np.uint8)
    blocks = [np.array([i]) for i in range(5)]  # one node per block: sequential Gibbs
    p = orc.Discrete(5, kinds, q, factors, blocks)
    ps, pc = _exact_marginals(3, 2, q, factors, p.energy)
    C = 6000
    sps, spc = _sampled_marginals(p, 3, 2, q, C, 60, 5)
    se_s = np.sqrt(ps * (1 - ps) / C)
    se_c = np.sqrt(pc * (1 - pc) / C)
    assert np.all(np.abs(sps - ps) < 5 * se_s + 1e-9), (sps, ps)
    assert np.all(np.abs(spc - pc) < 5 * se_c + 1e-9), (spc, pc)


def test_more_than_256_categories_exact_enumeration():
    """q = 300: a spin and a categorical node with a spin bias, a categorical
    bias and a spin-categorical factor; sampled marginals (one node per block,
    sequential Gibbs) against the exact distribution over all 2 x 300 states;
    results come back as uint16."""
    rng = np.random.default_rng(301)
    q = 300
    f = [([np.array([0])], [], rng.normal(0, 0.5, (1, 1, 1))),
         ([], [np.array([1])], rng.normal(0, 1.0, (1, q, 1))),
         ([np.array([0])], [np.array([1])], rng.normal(0, 1.0, (1, q, 1)))]
    factors = [(sg, cg, np.asarray(w, np.float32)) for sg, cg, w in f]
    p = orc.Discrete(2, np.array([0, 1], np.uint8), q, factors, [np.array([0]), np.array([1])])
    states = np.array([(s, x) for s in (0, 1) for x in range(q)], np.uint16)
    e = p.energy(states)
    w = np.exp(-(e - e.min()))
    w /= w.sum()
    exact_s = w[states[:, 0] == 1].sum()
    exact_x = np.array([w[states[:, 1] == c].sum() for c in range(q)])
    C = 8000
    st, _ = p.run_blocks(17, np.zeros((C, 2), np.uint16), 6)
    assert st.dtype == np.uint16 and st[:, 1].max() > 255
    got_x = np.bincount(st[:, 1], minlength=q) / C
    se_x = np.sqrt(exact_x * (1 - exact_x) / C) + 1e-9
    assert np.max(np.abs(got_x - exact_x) / se_x) < 5.5
    assert abs((st[:, 0] == 1).mean() - exact_s) < 5.5 * np.sqrt(exact_s * (1 - exact_s) / C)


@pytest.mark.parametrize("mistake", ["spin_sign", "swapped_axis"])
def test_planted_mistakes_move_the_marginals(mistake):
    """The exact marginals of the true model against the sampler of a model
    carrying a planted mistake: differences beyond 10 standard errors."""
    q, factors = _tiny()
    kinds = np.array([0, 0, 0, 1, 1], np.uint8)
    blocks = [np.array([i]) for i in range(5)]
    truth = orc.Discrete(5, kinds, q, factors, blocks)
    ps, pc = _exact_marginals(3, 2, q, factors, truth.energy)
    bad = list(factors)
    if mistake == "spin_sign":  # the three-body term with the opposite sign
        sg, cg, w = bad[1]
        bad[1] = (sg, cg, -w)
    else:  # the pair table transposed: the second head reads the wrong axis
        sg, cg, w = bad[4]
        bad[4] = (sg, cg, np.ascontiguousarray(np.transpose(w, (0, 2, 1))))
    wrong = orc.Discrete(5, kinds, q, bad, blocks)
    C = 6000
    sps, spc = _sampled_marginals(wrong, 3, 2, q, C, 60, 6)
    z_s = np.abs(sps - ps) / np.sqrt(ps * (1 - ps) / C)
    z_c = np.abs(spc - pc) / np.sqrt(pc * (1 - pc) / C)
    assert max(z_s.max(), z_c.max()) > 10


def test_spin_head_with_two_categorical_tails_reads_the_first():
    q = 3
    W = np.arange(1, 1 + q * q, dtype=np.float32).reshape(1, q, q)
    factors = [([np.array([0])], [np.array([1]), np.array([2])], W)]
    p = orc.Discrete(3, np.array([0, 1, 1], np.uint8), q, factors,
                     [np.array([0])], [np.array([1, 2])])
    for x1 in range(q):
        for x2 in range(q):
            st = np.array([1, x1, x2], np.uint8)
            assert p.params(st)[0, 0] == W.reshape(-1)[x1]


@pytest.mark.parametrize("factors,msg", [
    ([([], [], np.zeros((1, 1, 1), np.float32))], "At least one node group"),
    ([([np.array([0])], [], np.zeros((1, 2, 1), np.float32))], "weights \\[b, 1, 1\\]"),
    ([([], [np.array([2])], np.zeros((1, 1, 1), np.float32))], "effective dims"),
    ([([np.array([2])], [], np.zeros((1, 1, 1), np.float32))], "spin node groups must hold"),
    ([([], [np.array([2])], np.zeros((1, 2, 1), np.float32))], "weights \\[b, q, 1\\]"),
    ([([], [np.array([2]), np.array([3])], np.zeros((1, 3, 2), np.float32))], "weights \\[b, q, q\\]"),
])
def test_constructor_checks(factors, msg):
    kinds = np.array([0, 0, 1, 1], np.uint8)
    with pytest.raises(ValueError, match=msg):
        orc.Discrete(4, kinds, 3, factors, [np.array([0, 1]), np.array([2, 3])])


def test_block_of_two_kinds_is_rejected():
    with pytest.raises(ValueError, match="both spin and categorical"):
        orc.Discrete(2, np.array([0, 1], np.uint8), 3, [], [np.array([0, 1])])


def _square_case(seed, with_spins):
    """A square factor over categorical pairs drawn from one pool (nodes take
    both roles, several rows each), plus a bias factor; optional spin tails."""
    rng = np.random.default_rng(seed)
    q, n_spin, n_cat, m = 4, (12 if with_spins else 0), 30, 90
    n = n_spin + n_cat
    kinds = np.r_[np.zeros(n_spin), np.ones(n_cat)].astype(np.uint8)
    X = np.arange(n_spin, n)
    rows = [rng.choice(X, 2, replace=False) for _ in range(m)]
    U = np.array([r[0] for r in rows], np.uint32)
    V = np.array([r[1] for r in rows], np.uint32)
    W = rng.normal(0, 0.7, (m, q, q)).astype(np.float32)
    sg = [rng.choice(np.arange(n_spin), m).astype(np.uint32)] if with_spins else []
    free = ([np.arange(n_spin)] if with_spins else []) + [X[::2], X[1::2]]
    return rng, q, n, kinds, U, V, W, sg, free


@pytest.mark.parametrize("with_spins", [False, True])
def test_square_factor_merges_categorical_heads(with_spins):
    rng, q, n, kinds, U, V, W, sg, free = _square_case(11 + with_spins, with_spins)
    merged = orc.Discrete(n, kinds, q, [(sg, [U, V], W, True)], free)
    plain = orc.Discrete(n, kinds, q, [(sg, [U, V], W)], free)
    # shadow node of categorical node x: x + n_cat (a clamped block)
    n_sp = len(sg) and 12
    n_cat = n - n_sp
    X = np.arange(n_sp, n)
    WT = np.ascontiguousarray(W.transpose(0, 2, 1))
    shadow = orc.Discrete(n + n_cat, np.r_[kinds, np.ones(n_cat, np.uint8)], q,
                          [([np.r_[g, g] for g in sg], [np.r_[U, V], np.r_[V, U] + n_cat],
                            np.r_[W, WT])], free, [X + n_cat])
    shadow_pos = np.array([merged.pos(x) for x in X])
    differs = 0
    for _ in range(20):
        st = np.where(kinds == 0, rng.integers(0, 2, n), rng.integers(0, q, n)).astype(np.uint8)
        pm, pp = merged.params(st), plain.params(st)
        assert np.array_equal(pm[n_sp:], shadow.params(np.r_[st, st[shadow_pos]])[n_sp:])
        assert np.array_equal(pm[:n_sp], pp[:n_sp])
        assert np.allclose(pm, pp, rtol=0, atol=1e-5)
        differs += int((pm != pp).any())
        assert np.array_equal(merged.energy(st), plain.energy(st))
    assert differs > 0
    init = np.where(kinds[None] == 0, rng.integers(0, 2, (9, n)),
                    rng.integers(0, q, (9, n))).astype(np.uint8)
    a, _ = merged.run_blocks(5, init, 3)
    b, _ = plain.run_blocks(5, init, 3)
    assert (a != b).mean() < 1e-3  # the order changes decisions only at float32 ties


def test_square_factor_with_exact_weights_equals_unmerged():
    """Weights on a 1/8 grid: every sum is exact, so any order gives the same
    theta and the same samples as the unmerged factor."""
    rng, q, n, kinds, U, V, W, sg, free = _square_case(13, True)
    W = (np.round(W * 8) / 8).astype(np.float32)
    merged = orc.Discrete(n, kinds, q, [(sg, [U, V], W, True)], free)
    plain = orc.Discrete(n, kinds, q, [(sg, [U, V], W)], free)
    init = np.where(kinds[None] == 0, rng.integers(0, 2, (16, n)),
                    rng.integers(0, q, (16, n))).astype(np.uint8)
    assert np.array_equal(merged.run_blocks(9, init, 4)[0], plain.run_blocks(9, init, 4)[0])


def test_square_factor_shape_check():
    kinds = np.array([0, 0, 1, 1], np.uint8)
    blocks = [np.array([0, 1]), np.array([2, 3])]
    with pytest.raises(ValueError, match="Interaction tensor is not square"):
        orc.Discrete(4, kinds, 3, [([], [np.array([2]), np.array([3])],
                                    np.zeros((1, 3, 2), np.float32), True)], blocks)
    with pytest.raises(ValueError, match="Interaction tensor is not square"):
        orc.Discrete(4, kinds, 3, [([np.array([0])], [np.array([2])],
                                    np.zeros((1, 3, 1), np.float32), True)], blocks)
    # spin-only factors ([b, 1, 1]) are square: unchanged
    orc.Discrete(4, kinds, 3, [([np.array([0]), np.array([1])], [],
                                np.ones((1, 1, 1), np.float32), True)], blocks)
