"""MomentAccumulatorObserver with a general spec (crates/thrml-observers/src/
moment.rs:52-231) on every program kind, against the oracle's sample_states:
each row's sum over chains and observations of prod f(x), f(x) = 2x - 1 or x,
computed with numpy from the oracle's observed states (sampling.rs:178-320).

  - lattice and CSR Ising programs (1 and 2 chain groups), rows of 0 to 4
    nodes with repeats; the ising spec's rows equal thrml_moments' sums;
  - categorical and discrete factor programs, with and without the
    transform (category products);
  - a dense program against its own sample_states on the same key;
  - estimate_moments on a discrete program (through the general observer);
  - a node outside the program is rejected;
  - any AbstractObserver through sample_with_observation (a C callback per
    observation): it sees the states sample_states records, its carry
    accumulates the moment sums, a run started inside it is refused and an
    exception raised in it stops the run;
  - thrml_sample_states_as: the f32 observations equal the u8 ones on every
    program kind, and the u8 form refuses more than 256 categories."""
import numpy as np
import pytest

import pyoracle as orc
import thrml_hip as th
from conftest import log_case
from thrml_hip import workloads as wl

pytestmark = pytest.mark.gpu


def _expected(samples, pos_rows, transform):
    """sum over observations and chains of prod_k f(x[pos_k]) per row"""
    s = samples.astype(np.int64)
    f = 2 * s - 1 if transform else s
    out = []
    for rows in pos_rows:
        o = np.zeros(len(rows), np.int64)
        for i, r in enumerate(rows):
            prod = np.ones(f.shape[:2], np.int64)
            for p in r:
                prod *= f[:, :, p]
            o[i] = prod.sum()
        out.append(o)
    return out


def _rows(rng, nodes, n_types):
    types = [[[int(rng.choice(nodes))] for _ in range(30)],
             [[int(a), int(b)] for a, b in rng.choice(nodes, (30, 2))],
             [[int(x) for x in rng.choice(nodes, 3)] for _ in range(20)] + [[5, 5, 7]],
             [[int(x) for x in rng.choice(nodes, 4)] for _ in range(20)] + [[]]]
    return types[:n_types]


def _check(prog, spec, transform, key, sched, init):
    obs = th.MomentAccumulatorObserver(prog, spec, transform_to_spin=transform)
    st = prog.new_state(init.shape[0])
    st.set_global(init)
    got = obs.sample_with_observation(th.RngKey(key), th.SamplingSchedule(*sched), st)
    obs.close()
    st.close()
    return got


def _positions(o, rows_by_type):
    return [[[o.pos(n) for n in r] for r in t] for t in rows_by_type]


@pytest.mark.parametrize("transform", [True, False])
@pytest.mark.parametrize("kind,C", [("lattice", 64), ("csr", 100)])
def test_ising_programs(device, kind, C, transform):
    L = 32 if kind == "lattice" else 20
    ebm, blocks = wl.lattice_ising(L, 0.2, 0.3, 0.1)
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    assert prog.kind == kind
    o = orc.Ising(ebm.n_nodes, ebm.edges, ebm.biases, ebm.weights, ebm.beta,
                  [np.asarray(b.nodes if hasattr(b, "nodes") else b) for b in blocks])
    rng = np.random.default_rng(3)
    spec = _rows(rng, np.arange(ebm.n_nodes), 4)
    init = rng.integers(0, 2, (C, ebm.n_nodes)).astype(np.uint8)
    sched = (2, 5, 2)
    log_case(f"observer on {kind}, C={C}, transform={transform}")
    got = _check(prog, spec, transform, 11, sched, init)
    samples = o.sample_states(11, sched, init)
    want = _expected(samples, _positions(o, spec), transform)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)
    if transform:
        # the ising spec through the sweep kernels' own counters
        nodes = np.array([r[0] for r in spec[0]], np.uint32)
        pairs = np.array(spec[1], np.uint32)
        st = prog.new_state(C)
        st.set_global(init)
        ns, es = th.estimate_moments(th.RngKey(11), nodes, pairs, prog,
                                     th.SamplingSchedule(*sched), st, return_sums=True)
        assert np.array_equal(ns, got[0]) and np.array_equal(es, got[1])
        st.close()


@pytest.mark.parametrize("transform", [True, False])
@pytest.mark.parametrize("C", [40, 300])
def test_categorical_program(device, transform, C):
    n, edges, W, bias, blocks = wl.potts_lattice(16, 5, 0.3, 0.2)
    prog = th.CategoricalProgram(n, 5, edges, W, bias, blocks, device)
    o = orc.Potts(n, 5, edges, W, bias, [np.asarray(b.nodes if hasattr(b, "nodes") else b)
                                           for b in blocks])
    rng = np.random.default_rng(4)
    spec = _rows(rng, np.arange(n), 4)
    init = rng.integers(0, 5, (C, n)).astype(np.uint8)
    log_case(f"observer on a categorical program, transform={transform}, C={C}")
    got = _check(prog, spec, transform, 12, (1, 4, 3), init)
    want = _expected(o.sample_states(12, (1, 4, 3), init), _positions(o, spec), transform)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)


def _discrete(device, rng):
    q, ns, nc, m = 4, 60, 40, 50
    n = ns + nc
    kinds = np.r_[np.zeros(ns), np.ones(nc)].astype(np.uint8)
    S, X = np.arange(ns), np.arange(ns, n)
    f = [([S], [], rng.normal(0, 0.5, (ns, 1, 1))),
         ([rng.choice(S, m), rng.choice(S, m), rng.choice(S, m)], [], rng.normal(0, 0.5, (m, 1, 1))),
         ([rng.choice(S, m)], [rng.choice(X, m)], rng.normal(0, 0.5, (m, q, 1))),
         ([], [X], rng.normal(0, 0.5, (nc, q, 1)))]
    f = [(sg, cg, np.asarray(w, np.float32)) for sg, cg, w in f]
    free = [S[::2], S[1::2], X[::2], X[1::2]]
    prog = th.FactorSamplingProgram(kinds, q, [th.DiscreteEBMFactor(*x) for x in f], free, [],
                                    device)
    o = orc.Discrete(n, kinds, q, f, free)
    return q, n, kinds, free, prog, o


@pytest.mark.parametrize("transform", [True, False])
def test_discrete_program(device, transform):
    rng = np.random.default_rng(5)
    q, n, kinds, free, prog, o = _discrete(device, rng)
    spec = _rows(rng, np.arange(n), 4)
    order = np.concatenate(free)
    init = np.where(kinds[order][None] == 0, rng.integers(0, 2, (33, n)),
                    rng.integers(0, q, (33, n))).astype(np.uint8)
    log_case(f"observer on a discrete program, transform={transform}")
    got = _check(prog, spec, transform, 13, (2, 3, 2), init)
    want = _expected(o.sample_states(13, (2, 3, 2), init), _positions(o, spec), transform)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)


def test_estimate_moments_on_discrete_program(device):
    rng = np.random.default_rng(6)
    q, n, kinds, free, prog, o = _discrete(device, rng)
    nodes = np.arange(0, 60, 3, dtype=np.uint32)
    pairs = np.array([[0, 1], [2, 7], [10, 50]], np.uint32)
    order = np.concatenate(free)
    init = np.where(kinds[order][None] == 0, rng.integers(0, 2, (20, n)),
                    rng.integers(0, q, (20, n))).astype(np.uint8)
    st = prog.new_state(20)
    st.set_global(init)
    log_case("estimate_moments on a discrete program")
    ns, es = th.estimate_moments(th.RngKey(14), nodes, pairs, prog, th.SamplingSchedule(1, 6, 1),
                                 st, return_sums=True)
    samples = o.sample_states(14, (1, 6, 1), init)
    want = _expected(samples, [[[o.pos(x)] for x in nodes], [[o.pos(a), o.pos(b)] for a, b in pairs]],
                     True)
    assert np.array_equal(ns, want[0]) and np.array_equal(es, want[1])
    st.close()


def test_dense_program_against_its_own_states(device):
    bits, Wf, bv, bh = wl.rbm(64, 128, 0.1, 0.1)
    prog = th.RbmProgram(Wf, bv, bh, 1.0, device)
    rng = np.random.default_rng(7)
    spec = _rows(rng, np.arange(64 + 128), 3)
    st = th.hinton_init(th.RngKey(1), prog, 70)
    init = st.get_global()
    log_case("observer on a dense program")
    obs = th.MomentAccumulatorObserver(prog, spec)
    got = obs.sample_with_observation(th.RngKey(15), th.SamplingSchedule(1, 4, 2), st)
    st.set_global(init)
    samples = th.sample_states(th.RngKey(15), prog, th.SamplingSchedule(1, 4, 2), st)
    pos = [[[n for n in r] for r in t] for t in spec]  # dense: position = node id
    want = _expected(np.asarray(samples), pos, True)
    for g, w in zip(got, want):
        assert np.array_equal(g, w)
    obs.close()
    st.close()


def test_unknown_node_rejected(device):
    ebm, blocks = wl.lattice_ising(8, 0.1, 0.1, 0.1)
    prog = th.IsingSamplingProgram(ebm, blocks[:1], blocks[1:], device)
    with pytest.raises(th.ThrmlError, match="global location map"):
        th.MomentAccumulatorObserver(prog, [[[ebm.n_nodes + 3]]])


def test_categorical_rows_bounded_in_int64(device):
    """Category products are exact int64: a row whose product can exceed
    2^62 is refused at creation (q = 256: |2x - 1| <= 509, 509^7 > 2^62), and
    a run whose chains x observations x largest product could reach 2^63 is
    refused before it starts."""
    q = 256
    n, edges, W, bias, blocks = wl.potts_lattice(4, q, 0.2, 0.1)
    prog = th.CategoricalProgram(n, q, edges, W, bias, blocks, device)
    with pytest.raises(th.ThrmlError, match="can exceed int64"):
        th.MomentAccumulatorObserver(prog, [[list(range(7))]], transform_to_spin=True)
    th.MomentAccumulatorObserver(prog, [[list(range(7))]], transform_to_spin=False).close()
    obs = th.MomentAccumulatorObserver(prog, [[list(range(6))]], transform_to_spin=True)
    st = prog.new_state(300)  # 509^6 x 300 x 4 > 2^63
    with pytest.raises(th.ThrmlError, match="can exceed int64"):
        obs.sample_with_observation(th.RngKey(1), th.SamplingSchedule(1, 4, 1), st)
    obs.close()
    st.close()


class _Recorder(th.AbstractObserver):
    """Keeps every observed global state (the observation) and the running
    int64 sum of 2x - 1 per position (the carry)."""

    def init(self):
        return None

    def observe(self, state, carry, iteration):
        g = state.get_global()
        s = (2 * g.astype(np.int64) - 1).sum(0)
        return (s if carry is None else carry + s), (iteration, g)


@pytest.mark.parametrize("kind", ["lattice", "csr", "potts"])
def test_callback_observer_sees_sample_states(device, kind):
    log_case(f"callback observer {kind}")
    C, sched = 33, th.SamplingSchedule(2, 6, 3)
    if kind == "potts":
        n, edges, W, bias, blocks = wl.potts_lattice(8, 4, 0.5, 0.3, cfg=9)
        prog = th.CategoricalProgram(n, 4, edges, W, bias, blocks, device)
        init = np.random.default_rng(1).integers(0, 4, (C, n)).astype(np.uint8)
    else:
        ebm, blocks = wl.lattice_ising(32 if kind == "lattice" else 10, 0.1, 0.3, 0.05)
        prog = th.IsingSamplingProgram(ebm, blocks, [], device)
        assert prog.kind == kind
        init = np.random.default_rng(1).integers(0, 2, (C, ebm.n_nodes)).astype(np.uint8)
    st = prog.new_state(C)
    st.set_global(init)
    want = th.sample_states(th.RngKey(21), prog, sched, st)
    st.set_global(init)
    carry, obs = th.sample_with_observation(th.RngKey(21), prog, sched, st,
                                            f_observe=_Recorder())
    assert [i for i, _ in obs] == list(range(6))
    assert np.array_equal(np.stack([g for _, g in obs]), want)
    if kind != "potts":
        assert np.array_equal(carry, (2 * want.astype(np.int64) - 1).sum((0, 1)))


def test_callback_observer_refuses_nested_run_and_propagates_errors(device):
    log_case("callback observer errors")
    ebm, blocks = wl.lattice_ising(10, 0.1, 0.3, 0.05)
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    st = th.hinton_init(th.RngKey(2), prog, 8)

    class Nested(th.AbstractObserver):
        def observe(self, state, carry, iteration):
            th.run_blocks(th.RngKey(1), prog, state, (), 1)
            return carry, None

    with pytest.raises(th.ThrmlError, match="observer callback"):
        th.sample_with_observation(th.RngKey(3), prog, th.SamplingSchedule(1, 3, 1), st,
                                   f_observe=Nested())

    class Writes(th.AbstractObserver):
        def observe(self, state, carry, iteration):
            state.set_block(0, np.zeros((8, prog.block_range(0)[1]), np.uint8))
            return carry, None

    class Reinits(th.AbstractObserver):
        def observe(self, state, carry, iteration):
            th.hinton_init(th.RngKey(9), prog, state=state)
            return carry, None

    before = st.get_global()
    for obs in (Writes(), Reinits()):
        with pytest.raises(th.ThrmlError, match="observer callback"):
            th.sample_with_observation(th.RngKey(3), prog, th.SamplingSchedule(0, 1, 1), st,
                                       f_observe=obs)
        assert np.array_equal(st.get_global(), before)  # refused before any write

    class Fails(th.AbstractObserver):
        def observe(self, state, carry, iteration):
            if iteration == 2:
                raise ValueError("stop here")
            return (carry or 0) + 1, None

    with pytest.raises(ValueError, match="stop here"):
        th.sample_with_observation(th.RngKey(3), prog, th.SamplingSchedule(1, 5, 1), st,
                                   f_observe=Fails())
    # the context runs normally afterwards
    _, obs = th.sample_with_observation(th.RngKey(3), prog, th.SamplingSchedule(1, 4, 1), st,
                                        f_observe=_Recorder())
    assert [i for i, _ in obs] == [0, 1, 2, 3]


def _sample_states_as(prog, st, key, sched, dtype):
    import ctypes

    from thrml_hip import _lib

    n_obs = max(sched.n_samples, 1)
    out = np.zeros((n_obs, st.n_chains, prog.n_total),
                   np.float32 if dtype == _lib.DTYPE_F32 else np.uint8)
    rc = _lib.load().thrml_sample_states_as(prog._h, key, sched._c(), st._h,
                                            out.ctypes.data_as(ctypes.c_void_p), dtype)
    return rc, out


@pytest.mark.parametrize("kind", ["lattice", "csr", "dense", "potts", "discrete"])
def test_sample_states_f32_equals_u8(device, kind):
    """thrml_sample_states_as in the StateObserver's f32 representation
    writes the same observations as the u8 form, on every program kind."""
    from thrml_hip import _lib

    log_case(f"sample_states f32 vs u8 on {kind}")
    C, sched = 37, th.SamplingSchedule(2, 5, 2)
    rng = np.random.default_rng(4)
    if kind == "potts":
        n, edges, W, bias, blocks = wl.potts_lattice(8, 5, 0.5, 0.3, cfg=9)
        prog = th.CategoricalProgram(n, 5, edges, W, bias, blocks, device)
    elif kind == "discrete":
        n, kinds, fs, blocks = wl.mixed_lattice(8, 3)
        prog = th.FactorSamplingProgram(kinds, 3, fs, blocks, [], device)
    elif kind == "dense":
        _, Wf, bv, bh = wl.rbm(64, 128, 0.1, 0.1)
        prog = th.RbmProgram(Wf, bv, bh, 1.0, device)
    else:
        ebm, blocks = wl.lattice_ising(32 if kind == "lattice" else 10, 0.1, 0.3, 0.05)
        prog = th.IsingSamplingProgram(ebm, blocks, [], device)
        assert prog.kind == kind
    if kind in ("lattice", "csr", "dense"):
        st = th.hinton_init(th.RngKey(3), prog, C)
    else:
        st = prog.new_state(C)
        hi = np.where(np.asarray(kinds) == 1, 3, 2) if kind == "discrete" else 5
        st.set_global(rng.integers(0, hi, (C, prog.n_total)).astype(np.uint8))
    init = st.get_global()
    rc, u8 = _sample_states_as(prog, st, 9, sched, _lib.DTYPE_U8)
    assert rc == 0
    st.set_global(init)
    rc, f32 = _sample_states_as(prog, st, 9, sched, _lib.DTYPE_F32)
    assert rc == 0
    assert np.array_equal(f32, u8.astype(np.float32))
    st.set_global(init)
    assert np.array_equal(th.sample_states(th.RngKey(9), prog, sched, st), u8)
    st.close()


def test_sample_states_u8_refuses_more_than_256_categories(device):
    """The u8 form refuses a two-byte categorical state (categories above 255
    do not fit), the f32 form takes it, and an unknown dtype is refused."""
    from thrml_hip import _lib

    from test_gpu_potts import _ring

    log_case("sample_states dtype errors")
    q, n = 300, 8
    _, edges, W, bias = _ring(n, q, 9)
    prog = th.CategoricalProgram(n, q, edges, W, bias, [np.arange(n)], device)
    st = prog.new_state(4)
    sched = th.SamplingSchedule(1, 2, 1)
    rc, _ = _sample_states_as(prog, st, 1, sched, _lib.DTYPE_U8)
    assert rc == _lib.THRML_EINVAL and "u8 dtype" in _lib.load().thrml_last_error().decode()
    rc, f = _sample_states_as(prog, st, 1, sched, _lib.DTYPE_F32)
    assert rc == 0 and f.shape == (2, 4, n) and (f == np.round(f)).all() and f.max() < q
    rc, _ = _sample_states_as(prog, st, 1, sched, 7)
    assert rc == _lib.THRML_EINVAL
    st.close()
