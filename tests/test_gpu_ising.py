"""GPU parity of the Ising sweep (libthrml_hip.so through the C ABI) against
the CPU oracle: bit-identical states for the same RngKey and schedule, exact
moment sums.  Cases: config 1 at its full size, a full-size 1024^2 lattice on
a subset of chains, CSR programs with clamped blocks, intra-block edges and
chain counts that are not multiples of 64, the kernel-level exports."""
import numpy as np
import pytest

import pyoracle as orc
import thrml_hip as th
from conftest import log_case
from thrml_hip import workloads as wl

pytestmark = pytest.mark.gpu


def _oracle_prog(ebm, free_blocks, clamped=()):
    return orc.Ising(ebm.n_nodes, ebm.edges, ebm.biases, ebm.weights, ebm.beta,
                     [b.nodes if hasattr(b, "nodes") else b for b in free_blocks],
                     [b.nodes if hasattr(b, "nodes") else b for b in clamped])


def test_state_roundtrip(device):
    log_case("state_roundtrip C=130")
    ebm, blocks = wl.lattice_ising(8, 0.1, 0.3, 0.05)
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    st = prog.new_state(130)
    rng = np.random.default_rng(0)
    for b in range(2):
        v = rng.integers(0, 2, (130, 32)).astype(np.uint8)
        st.set_block(b, v)
        assert np.array_equal(st.get_block(b), v)
        st.set_block(b, v.astype(np.float32))
        assert np.array_equal(st.get_block(b, np.float32), v.astype(np.float32))


def test_sigmoid_bernoulli_and_gumbel_exports(device):
    import ctypes

    import torch

    from thrml_hip import _lib

    log_case("kernel exports")
    rng = np.random.default_rng(1)
    n = 1 << 16
    g = rng.normal(0, 3, n).astype(np.float32)
    u = rng.random(n).astype(np.float32)
    gd, ud = torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda()
    od = torch.empty(n, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    _lib.check(_lib.load().thrml_sigmoid_bernoulli(device.handle, ctypes.c_void_p(gd.data_ptr()),
                                                   ctypes.c_void_p(ud.data_ptr()),
                                                   ctypes.c_void_p(od.data_ptr()), n))
    device.synchronize()
    want = (u < orc.map_f32("sigmoid", 2.0 * g)).astype(np.float32)
    assert np.array_equal(od.cpu().numpy(), want)
    q = 8
    logits = rng.normal(0, 1, (4096, q)).astype(np.float32)
    uu = rng.uniform(1e-6, 1 - 1e-6, (4096, q)).astype(np.float32)
    ld, ud2 = torch.from_numpy(logits).cuda(), torch.from_numpy(uu).cuda()
    o2 = torch.empty(4096, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    _lib.check(_lib.load().thrml_gumbel_argmax(device.handle, ctypes.c_void_p(ld.data_ptr()),
                                               ctypes.c_void_p(ud2.data_ptr()),
                                               ctypes.c_void_p(o2.data_ptr()), 4096, q))
    device.synchronize()
    pert = logits - orc.map_f32("log", -orc.map_f32("log", uu.ravel())).reshape(4096, q)
    assert np.array_equal(o2.cpu().numpy(), np.argmax(pert, axis=1))


def test_config1_full_parity(device):
    """64^2 torus, 256 chains, hinton init, 1000 sweeps, RngKey(42): identical states."""
    c = wl.CONFIGS[1]
    ebm, blocks = wl.config_ising(1)
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    assert prog.kind == "lattice"
    k_init, k_run = th.RngKey(c["key"]).split_two()
    log_case("config1 hinton")
    st = th.hinton_init(k_init, prog, c["chains"])
    o = _oracle_prog(ebm, blocks)
    init = o.hinton_init(k_init.seed, c["chains"])
    assert np.array_equal(st.get_global(), init)
    log_case("config1 1000 sweeps")
    th.run_blocks(k_run, prog, st, (), c["sweeps"])
    got = st.get_global()
    want, near = o.run_blocks(k_run.seed, init, c["sweeps"])
    print(f"threshold sites (|2g - logit u| < 1e-5) in the oracle run: {near}")
    assert np.array_equal(got, want)


def test_lattice_full_size_chain_subset(device):
    """1024^2 torus (config 2 shape), 64 chains, 6 sweeps: chains 0, 17, 63 vs oracle."""
    ebm, blocks = wl.config_ising(2)
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    assert prog.kind == "lattice"
    log_case("config2 shape, 6 sweeps")
    st = th.hinton_init(th.RngKey(5), prog, 64)
    init = st.get_global()
    th.run_blocks(th.RngKey(42), prog, st, (), 6)
    got = st.get_global()
    o = _oracle_prog(ebm, blocks)
    sel = [0, 17, 63]
    want = o.run_blocks_subset(42, 64, sel, init[sel], 6)
    assert np.array_equal(got[sel], want)


def test_config3_full_size_all_chains(device):
    """Config 3 at full size (Erdos-Renyi 1M nodes, mean degree 12, greedy
    colouring into 10 blocks, 32 chains), 2 sweeps: every chain against the
    oracle.  Its blocks take the three 4-site-run kernels (regions of up to 32
    and 40 slots, and the general staging)."""
    log_case("config3 full size, 2 sweeps, all 32 chains")
    ebm, blocks = wl.config3()
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    assert prog.kind == "csr"
    st = th.hinton_init(th.RngKey(3), prog, 32)
    init = st.get_global()
    th.run_blocks(th.RngKey(43), prog, st, (), 2)
    got = st.get_global()
    want, near = _oracle_prog(ebm, blocks).run_blocks(43, init, 2)
    print(f"threshold sites in the oracle run: {near}")
    assert np.array_equal(got, want)


@pytest.mark.parametrize("L,C,sweeps", [(4, 1, 50), (6, 65, 20), (32, 64, 40), (10, 200, 15),
                                         (32, 1, 30), (64, 130, 12), (96, 37, 10)])
def test_lattice_small_parity(device, L, C, sweeps):
    """Lattice programs; L % 32 == 0 takes the lattice kernel, others the CSR kernel."""
    log_case(f"lattice L={L} C={C}")
    ebm, blocks = wl.lattice_ising(L, 0.3, 0.2, 0.5)
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    assert prog.kind == ("lattice" if L % 32 == 0 else "csr")
    rng = np.random.default_rng(L * 1000 + C)
    init = rng.integers(0, 2, (C, L * L)).astype(np.uint8)
    st = prog.new_state(C)
    st.set_global(init)
    th.run_blocks(th.RngKey(L + C), prog, st, (), sweeps)
    want, _ = _oracle_prog(ebm, blocks).run_blocks(L + C, init, sweeps)
    assert np.array_equal(st.get_global(), want)


def _random_program(n, m, n_free, n_clamp, seed, intra=False):
    rng = np.random.default_rng(seed)
    perm = rng.permutation(n)
    cuts = np.sort(rng.choice(np.arange(1, n), n_free + n_clamp - 1, replace=False))
    parts = np.split(perm, cuts)
    edges = set()
    while len(edges) < m:
        a, b = (int(x) for x in rng.integers(0, n, 2))
        if a != b:
            edges.add((a, b))
    edges = np.array(sorted(edges), np.uint32)
    b = rng.normal(0, 0.5, n).astype(np.float32)
    w = rng.normal(0, 0.6, edges.shape[0]).astype(np.float32)
    ebm = th.IsingEBM(n, edges, b, w, 0.9)
    return ebm, parts[:n_free], parts[n_free:]


@pytest.mark.parametrize("C", [1, 37, 64, 130])
def test_csr_parity_with_clamped_and_intra_block_edges(device, C):
    log_case(f"csr C={C}")
    ebm, free, clamped = _random_program(300, 900, 4, 1, seed=C)
    prog = th.IsingSamplingProgram(ebm, free, clamped, device)
    assert prog.kind == "csr"
    rng = np.random.default_rng(C + 1)
    init = rng.integers(0, 2, (C, prog.n_total)).astype(np.uint8)
    st = prog.new_state(C)
    st.set_global(init)
    th.run_blocks(th.RngKey(3 * C), prog, st, (), 12)
    want, _ = _oracle_prog(ebm, free, clamped).run_blocks(3 * C, init, 12)
    got = st.get_global()
    assert np.array_equal(got, want)
    off, n = prog.block_range(len(free))
    assert np.array_equal(got[:, off:off + n], init[:, off:off + n])  # clamped block untouched


def _edges_program(n, edges, seed, blocks=None):
    rng = np.random.default_rng(seed)
    edges = np.unique(np.asarray(edges, np.uint32), axis=0)
    edges = edges[edges[:, 0] != edges[:, 1]]
    b = rng.normal(0, 0.3, n).astype(np.float32)
    w = rng.normal(0, 0.4, edges.shape[0]).astype(np.float32)
    ebm = th.IsingEBM(n, edges, b, w, 1.0)
    if blocks is None:
        blocks = th.coloring_to_blocks(th.greedy_coloring(n, edges))
    return ebm, blocks


@pytest.mark.parametrize("C,na", [(32, 140000), (64, 140000), (100, 140000), (32, 80000),
                                  (64, 40000)])
def test_csr_large_blocks(device, C, na):
    """Two blocks of na sites.  The launch takes 16-site runs (two runs per
    wave at <= 32 chains) from 4096 waves of them up, else 4-site runs:
    140000 sites give 16-site runs, 80000 (two runs per wave) and 40000 (64
    chains) 4-site runs over thousands of waves."""
    log_case(f"csr bipartite 2x{na} C={C}")
    rng = np.random.default_rng(C + na)
    e = np.stack([rng.integers(0, na, 4 * na), na + rng.integers(0, na, 4 * na)], 1)
    ebm, blocks = _edges_program(2 * na, e, C, [np.arange(na), np.arange(na, 2 * na)])
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    assert prog.kind == "csr"
    init = rng.integers(0, 2, (C, 2 * na)).astype(np.uint8)
    st = prog.new_state(C)
    st.set_global(init)
    th.run_blocks(th.RngKey(C + 5), prog, st, (), 2)
    want, _ = _oracle_prog(ebm, blocks).run_blocks(C + 5, init, 2)
    assert np.array_equal(st.get_global(), want)


@pytest.mark.parametrize("C,clamp", [(7, False), (32, False), (33, False), (20, True)])
def test_csr_runs_after_state_writes(device, C, clamp):
    """Runs interleaved with state writes: with at most 32 chains the sweeps
    gather from a half-size copy of the state that each run refreshes from
    the words, so a block written between runs (and a whole new state) must
    reach the next run's first sweep.  33 chains take the 64-chain words.
    clamp: the last colour class is a clamped block, and the block written
    between runs is that one (as a training loop writes its data rows)."""
    log_case(f"csr runs after writes C={C} clamp={clamp}")
    n = 20000
    rng = np.random.default_rng(40 + C)
    ebm, blocks = _edges_program(n, rng.integers(0, n, (6 * n, 2)), C)
    free, clamped = (blocks[:-1], blocks[-1:]) if clamp else (blocks, [])
    prog = th.IsingSamplingProgram(ebm, free, clamped, device)
    assert prog.kind == "csr"
    o = _oracle_prog(ebm, free, clamped)
    want = rng.integers(0, 2, (C, n)).astype(np.uint8)
    st = prog.new_state(C)
    st.set_global(want)
    th.run_blocks(th.RngKey(C + 1), prog, st, (), 3)
    want, _ = o.run_blocks(C + 1, want, 3)
    assert np.array_equal(st.get_global(), want)
    # one block rewritten, then a second run
    wb = len(free) if clamp else 1
    off, nb = prog.block_range(wb)
    vals = rng.integers(0, 2, (C, nb)).astype(np.uint8)
    st.set_block(wb, vals)
    want[:, off:off + nb] = vals
    th.run_blocks(th.RngKey(C + 2), prog, st, (), 2)
    want, _ = o.run_blocks(C + 2, want, 2)
    assert np.array_equal(st.get_global(), want)
    # two runs back to back, then a whole new state
    th.run_blocks(th.RngKey(C + 3), prog, st, (), 1)
    th.run_blocks(th.RngKey(C + 4), prog, st, (), 1)
    want, _ = o.run_blocks(C + 3, want, 1)
    want, _ = o.run_blocks(C + 4, want, 1)
    assert np.array_equal(st.get_global(), want)
    want = rng.integers(0, 2, (C, n)).astype(np.uint8)
    st.set_global(want)
    th.run_blocks(th.RngKey(C + 5), prog, st, (), 2)
    want, _ = o.run_blocks(C + 5, want, 2)
    assert np.array_equal(st.get_global(), want)
    # hinton_init into the same state, then a run
    th.hinton_init(th.RngKey(C + 6), prog, state=st)
    want = o.hinton_init(C + 6, C)
    if clamp:  # hinton_init draws the free blocks; the clamped block is set
        vals = rng.integers(0, 2, (C, nb)).astype(np.uint8)
        st.set_block(wb, vals)
        want[:, off:off + nb] = vals
    assert np.array_equal(st.get_global(), want)
    th.run_blocks(th.RngKey(C + 7), prog, st, (), 2)
    want, _ = o.run_blocks(C + 7, want, 2)
    assert np.array_equal(st.get_global(), want)
    st.close()


@pytest.mark.parametrize("C", [5, 64])
def test_csr_high_degree_sites(device, C):
    """Mean degree ~150 (several staging passes per wave) and a hub with 3000
    neighbours (its wave's slots exceed the LDS stage: read from global memory)."""
    log_case(f"csr hub C={C}")
    n = 4000
    rng = np.random.default_rng(7 + C)
    hub = np.stack([np.zeros(3000, np.int64), np.arange(1, 3001)], 1)
    e = np.concatenate([hub, rng.integers(0, n, (300000, 2))])
    ebm, blocks = _edges_program(n, e, C)
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    assert prog.kind == "csr"
    init = rng.integers(0, 2, (C, n)).astype(np.uint8)
    st = prog.new_state(C)
    st.set_global(init)
    th.run_blocks(th.RngKey(C + 9), prog, st, (), 3)
    want, _ = _oracle_prog(ebm, blocks).run_blocks(C + 9, init, 3)
    assert np.array_equal(st.get_global(), want)


@pytest.mark.parametrize("hub_deg,C", [(28, 32), (33, 1), (36, 32), (40, 17), (41, 32), (100, 20)])
def test_csr_half_site_regions(device, hub_deg, C):
    """Up to 32 chains, sites take per-site LDS regions: a sparse graph (mean
    degree 8, largest about 22) where 12 hubs get exactly hub_deg neighbours.
    Blocks whose sites have at most 32 or 40 slots run the region-only
    kernels; above 40 the general kernel mixes region waves with waves whose
    hub takes the masked path."""
    log_case(f"csr half regions hub_deg={hub_deg} C={C}")
    n = 30000
    rng = np.random.default_rng(hub_deg * 100 + C)
    e = rng.integers(0, n, (4 * n, 2)).astype(np.uint32)
    e = np.unique(np.sort(e, axis=1), axis=0)
    e = e[e[:, 0] != e[:, 1]]
    for hub in rng.choice(n, 12, replace=False):
        deg = np.bincount(e.reshape(-1), minlength=n)
        adj = set(e[e[:, 0] == hub, 1]) | set(e[e[:, 1] == hub, 0]) | {hub}
        cand = np.array([v for v in rng.permutation(n)[:4 * hub_deg] if v not in adj])
        k = hub_deg - int(deg[hub])
        add = np.sort(np.stack([np.full(k, hub), cand[:k]], 1), axis=1).astype(np.uint32)
        e = np.unique(np.concatenate([e, add]), axis=0)
    ebm, blocks = _edges_program(n, e, C)
    deg = np.bincount(np.asarray(ebm.edges).reshape(-1), minlength=n)
    assert hub_deg <= deg.max() <= hub_deg + 2  # (a later hub may join an earlier one)
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    assert prog.kind == "csr"
    init = rng.integers(0, 2, (C, n)).astype(np.uint8)
    st = prog.new_state(C)
    st.set_global(init)
    th.run_blocks(th.RngKey(C + hub_deg), prog, st, (), 3)
    want, _ = _oracle_prog(ebm, blocks).run_blocks(C + hub_deg, init, 3)
    assert np.array_equal(st.get_global(), want)


def test_lattice_with_reordered_block_takes_csr_path(device):
    log_case("lattice reordered -> csr")
    ebm, (up, lo) = wl.lattice_ising(16, 0.1, 0.3, 0.05)
    blocks = [up.nodes[::-1].copy(), lo.nodes]
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    assert prog.kind == "csr"
    init = np.random.default_rng(2).integers(0, 2, (64, 256)).astype(np.uint8)
    st = prog.new_state(64)
    st.set_global(init)
    th.run_blocks(th.RngKey(1), prog, st, (), 25)
    want, _ = _oracle_prog(ebm, blocks).run_blocks(1, init, 25)
    assert np.array_equal(st.get_global(), want)


@pytest.mark.parametrize("kind,sched,pairs", [
    ("lattice", (3, 40, 2), "edges"),      # counts fused into the sweep kernel
    ("lattice", (0, 7, 3), "edges"),       # first observation precedes every sweep
    ("lattice", (2, 5, 0), "edges"),       # repeated observations of one state
    ("lattice", (1, 9, 1), "reversed"),    # edges given as (v, u), shuffled
    ("lattice", (2, 6, 2), "mixed"),       # a non-edge pair: per-entry counters
    ("csr", (3, 40, 2), "edges"),
])
def test_moments_parity(device, kind, sched, pairs):
    log_case(f"moments {kind} {sched} {pairs}")
    if kind == "lattice":
        ebm, blocks = wl.lattice_ising(32, 0.1, 0.44, 0.05)
        clamped = []
    else:
        ebm, blocks, clamped = _random_program(200, 600, 3, 1, seed=9)
    prog = th.IsingSamplingProgram(ebm, blocks, clamped, device)
    assert prog.kind == kind
    C = 96
    init = np.random.default_rng(4).integers(0, 2, (C, prog.n_total)).astype(np.uint8)
    nodes = np.arange(ebm.n_nodes)
    e = ebm.edges.copy()
    rng = np.random.default_rng(11)
    if pairs == "reversed":
        e = e[rng.permutation(e.shape[0])][:, ::-1].copy()
        nodes = rng.permutation(nodes)[:300]
    elif pairs == "mixed":
        e = np.concatenate([e, [[0, 2], [5, 5]]]).astype(np.uint32)
    st = prog.new_state(C)
    st.set_global(init)
    ns, es = th.estimate_moments(th.RngKey(42), nodes, e, prog, th.SamplingSchedule(*sched), st,
                                 return_sums=True)
    o = _oracle_prog(ebm, blocks, clamped)
    ons, oes, ofinal, _ = o.estimate_moments(42, sched, init, nodes, e)
    assert np.array_equal(ns, ons)
    assert np.array_equal(es, oes)
    assert np.array_equal(st.get_global(), ofinal)


def test_sample_states_consistent_with_moments(device):
    log_case("sample_states")
    ebm, blocks = wl.lattice_ising(8, 0.2, 0.3, 0.1)
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    C = 70
    init = np.random.default_rng(5).integers(0, 2, (C, 64)).astype(np.uint8)
    sched = th.SamplingSchedule(2, 6, 3)
    st = prog.new_state(C)
    st.set_global(init)
    samples = th.sample_states(th.RngKey(8), prog, sched, st)
    assert samples.shape == (6, C, 64)
    st2 = prog.new_state(C)
    st2.set_global(init)
    ns, es = th.estimate_moments(th.RngKey(8), np.arange(64), ebm.edges, prog, sched, st2,
                                 return_sums=True)
    t = 2 * samples.astype(np.int64) - 1
    pos = [prog_pos for prog_pos in range(64)]
    glob_of_node = np.empty(64, np.int64)
    for b in range(2):
        off, n = prog.block_range(b)
        glob_of_node[blocks[b].nodes] = np.arange(off, off + n)
    assert np.array_equal(t[:, :, glob_of_node].sum(axis=(0, 1)), ns)
    e = ebm.edges
    assert np.array_equal((t[:, :, glob_of_node[e[:, 0]]] * t[:, :, glob_of_node[e[:, 1]]]).sum(axis=(0, 1)), es)
    del pos


@pytest.mark.parametrize("C", [1, 37])
def test_sample_states_matches_oracle(device, C):
    """Whole-state samples equal the oracle's at every observation, and
    nodes_to_sample returns the reference's per-block float32 arrays
    (sampling.rs:128-156): [n_samples, len] for one chain, gathered by node
    (a block in another order, a node of a clamped block)."""
    log_case(f"sample_states vs oracle C={C}")
    edges = np.array([(i, (i * 7 + 3) % 90) for i in range(90) if (i * 7 + 3) % 90 != i], np.uint32)
    rng = np.random.default_rng(C)
    b = rng.normal(0, 0.4, 90).astype(np.float32)
    w = rng.normal(0, 0.5, edges.shape[0]).astype(np.float32)
    ebm = th.IsingEBM(90, edges, b, w, 0.7)
    free = [np.arange(0, 80, 2), np.arange(1, 80, 2)]
    clamped = [np.arange(80, 90)]
    prog = th.IsingSamplingProgram(ebm, [th.Block(f) for f in free], [th.Block(clamped[0])], device)
    init = rng.integers(0, 2, (C, prog.n_total)).astype(np.uint8)
    st = prog.new_state(C)
    st.set_global(init)
    sched = th.SamplingSchedule(2, 4, 3)
    got = th.sample_states(th.RngKey(31), prog, sched, st)
    want = orc.Ising(90, edges, b, w, 0.7, free, clamped).sample_states(31, (2, 4, 3), init)
    assert np.array_equal(got, want)
    blk_a = th.Block(np.array([5, 3, 1, 84, 0]))
    blk_b = th.Block(np.arange(10, 30))
    st.set_global(init)
    per = th.sample_states(th.RngKey(31), prog, sched, st, nodes_to_sample=[blk_a, blk_b])
    pos = np.empty(90, np.int64)
    for k in range(3):
        off, n = prog.block_range(k)
        pos[(free + clamped)[k]] = np.arange(off, off + n)
    for blk, arr in zip([blk_a, blk_b], per):
        assert arr.dtype == np.float32
        ref = want[:, :, pos[blk.nodes]].astype(np.float32)
        assert np.array_equal(arr, ref[:, 0, :] if C == 1 else ref)
    with pytest.raises(th.ThrmlError):
        th.sample_states(th.RngKey(31), prog, sched, st, nodes_to_sample=[th.Block(np.array([95]))])


def test_energy_matches_oracle(device):
    ebm, blocks = wl.lattice_ising(8, 0.2, 0.3, 0.1)
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    init = np.random.default_rng(6).integers(0, 2, (5, 64)).astype(np.uint8)
    st = prog.new_state(5)
    st.set_global(init)
    assert np.allclose(th.ising_energy(prog, st), _oracle_prog(ebm, blocks).energy(init))


def test_error_behaviour(device):
    ebm, blocks = wl.lattice_ising(4, 0.1, 0.3, 0.05)
    with pytest.raises(th.ThrmlError, match="twice"):
        th.IsingSamplingProgram(ebm, [blocks[0].nodes, blocks[0].nodes], [], device)
    with pytest.raises(th.ThrmlError, match="global location map"):
        th.IsingSamplingProgram(ebm, [blocks[0].nodes], [], device)
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    other = th.IsingSamplingProgram(ebm, blocks, [], device)
    st = other.new_state(3)
    with pytest.raises(th.ThrmlError, match="another program"):
        th.run_blocks(th.RngKey(1), prog, st, (), 1)
    with pytest.raises(th.ThrmlError, match="out of range"):
        st.get_block(5)
    # n_iters = 0 is the identity (sampling.rs:89-91)
    st2 = prog.new_state(3)
    st2.set_global(np.ones((3, 16), np.uint8))
    th.run_blocks(th.RngKey(1), prog, st2, (), 0)
    assert st2.get_global().all()
    # the raw C ABI: blocks announced with NULL arrays are an error, not a read
    import ctypes

    from thrml_hip import _lib

    b = np.zeros(16, np.float32)
    d = _lib.IsingDesc(16, 0, None, None, _lib.ptr(b, ctypes.c_float), None, 1.0, 1, None, None,
                       0, None, None)
    h = ctypes.c_void_p()
    rc = _lib.load().thrml_ising_program_create(device.handle, ctypes.byref(d), ctypes.byref(h))
    assert rc == _lib.THRML_EINVAL and b"NULL" in _lib.load().thrml_last_error()


@pytest.mark.parametrize("kind", ["lattice", "csr"])
def test_observer_reuse_and_device_output(device, kind):
    """A MomentAccumulatorObserver built once serves several runs; sums written
    to device tensors equal the host sums and the oracle's."""
    import torch

    log_case(f"observer reuse {kind}")
    if kind == "lattice":
        ebm, blocks = wl.lattice_ising(64, 0.1, 0.44, 0.05)
        clamped = []
    else:
        ebm, blocks, clamped = _random_program(150, 500, 3, 0, seed=21)
    prog = th.IsingSamplingProgram(ebm, blocks, clamped, device)
    assert prog.kind == kind
    C = 70
    init = np.random.default_rng(8).integers(0, 2, (C, prog.n_total)).astype(np.uint8)
    nodes = np.arange(ebm.n_nodes, dtype=np.uint32)
    obs = th.MomentAccumulatorObserver(prog, th.ising_moment_spec(nodes, ebm.edges))
    st = prog.new_state(C)
    st.set_global(init)
    o = _oracle_prog(ebm, blocks, clamped)
    state = init
    for i, sched in enumerate([(2, 9, 3), (1, 17, 1)]):
        ns, es = obs.sample_with_observation(th.RngKey(100 + i), th.SamplingSchedule(*sched), st)
        ons, oes, state, _ = o.estimate_moments(100 + i, sched, state, nodes, ebm.edges)
        assert np.array_equal(ns, ons) and np.array_equal(es, oes)
    st.set_global(init)
    a = torch.full((nodes.size,), -7, dtype=torch.int64, device="cuda")
    b = torch.full((ebm.edges.shape[0],), -7, dtype=torch.int64, device="cuda")
    torch.cuda.synchronize()
    obs.sample_with_observation(th.RngKey(100), th.SamplingSchedule(2, 9, 3), st, out=(a, b))
    device.synchronize()
    ons, oes, _, _ = o.estimate_moments(100, (2, 9, 3), init, nodes, ebm.edges)
    assert np.array_equal(a.cpu().numpy(), ons) and np.array_equal(b.cpu().numpy(), oes)
    obs.close()


@pytest.mark.parametrize("span", [False, True])
def test_kernel_timing_counts_launches(device, span):
    """Both timing modes count one sweep launch per block per sweep and give
    a positive average; turning timing off resets them."""
    log_case(f"kernel timing span={span}")
    ebm, blocks = wl.lattice_ising(32, 0.2, 0.3, 0.1)
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    st = prog.new_state(64)
    device.enable_timing(True, span=span)
    th.run_blocks(th.RngKey(3), prog, st, (), 7)
    ms, n = device.kernel_time(0)
    assert n == 14 and ms > 0
    device.enable_timing(False)
    assert device.kernel_time(0) == (0.0, 0)


def test_state_outlives_program(device):
    """A state and a moment specification destroyed after their program (as
    when a training spec is closed while its hinton states are still held)."""
    log_case("state outlives program")
    ebm, blocks = wl.lattice_ising(8, 0.2, 0.3, 0.1)
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    st = prog.new_state(5)
    obs = th.MomentAccumulatorObserver(prog, th.ising_moment_spec(np.arange(64), ebm.edges))
    prog.close()
    with pytest.raises(th.ThrmlError):
        th.run_blocks(th.RngKey(1), prog, st, (), 1)
    obs.close()
    st.close()
