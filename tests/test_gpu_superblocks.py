"""Superblocks on the device (BlockGibbsSpec::new,
crates/thrml-samplers/src/program.rs:28-64; sample_blocks,
crates/thrml-samplers/src/sampling.rs:28-63) against the oracle, bit for bit:

  - Ising (CSR kernel) with grouped blocks, one superblock over every free
    block (a synchronous sweep) next to a clamped block, blocks with edges
    inside them, empty superblocks; both chain layouts (C <= 32 and
    several groups of 64);
  - a torus lattice and a complete bipartite model with grouped blocks leave
    the lattice and matrix-core kernels for the CSR kernel, and still match;
  - categorical programs with grouped blocks, clamped blocks and edges
    inside blocks; sample_states and estimate_moments through the schedule;
  - thrml_run_blocks_noalloc on a grouped program equals thrml_run_blocks;
  - the Python API's nested superblock lists, and the rejection of offsets
    that are not a partition of the free blocks."""
import numpy as np
import pytest

import pyoracle as orc
import thrml_hip as th
from conftest import log_case
from thrml_hip import _lib
from thrml_hip import workloads as wl

pytestmark = pytest.mark.gpu


def _graph(n, m, seed):
    rng = np.random.default_rng(seed)
    e = set()
    while len(e) < m:
        a, b = (int(v) for v in rng.integers(0, n, 2))
        if a != b:
            e.add((a, b))
    edges = np.array(sorted(e), np.uint32)
    return rng, edges


def _coloured_blocks(n, edges):
    col, _ = orc.greedy_coloring(n, edges)
    return [np.nonzero(col == c)[0].astype(np.uint32) for c in range(int(col.max()) + 1)]


def _nest(blocks, off):
    """Superblock offsets -> the nested list IsingSamplingProgram takes."""
    return [[blocks[b] for b in range(off[s], off[s + 1])] for s in range(len(off) - 1)]


def _ising_case(device, n, edges, b, w, beta, free, clamped, off, C, n_iters, seed, key):
    ebm = th.IsingEBM(n, edges, b, w, beta)
    prog = th.IsingSamplingProgram(ebm, _nest(free, off), clamped, device)
    o = orc.Ising(n, edges, b, w, beta, free, clamped, superblocks=off)
    init = np.random.default_rng(seed).integers(0, 2, (C, prog.n_total)).astype(np.uint8)
    st = prog.new_state(C)
    st.set_global(init)
    th.run_blocks(th.RngKey(key), prog, st, (), n_iters)
    got = st.get_global()
    want, _ = o.run_blocks(key, init, n_iters)
    st.close()
    return prog, got, want


@pytest.mark.parametrize("C", [5, 64, 150])
def test_ising_grouped_blocks(device, C):
    n = 300
    rng, edges = _graph(n, 900, 1)
    b = rng.normal(0, 0.4, n).astype(np.float32)
    w = rng.normal(0, 0.6, len(edges)).astype(np.float32)
    blocks = _coloured_blocks(n, edges)
    nb = len(blocks)
    assert nb >= 4
    off = [0, 2, 3, nb]  # {0, 1}, {2}, {3 .. nb-1}
    log_case(f"ising grouped blocks n={n} blocks={nb} superblocks={off} C={C}")
    prog, got, want = _ising_case(device, n, edges, b, w, 1.1, blocks, [], off, C, 4, 2, 33)
    assert prog.kind == "csr"
    assert prog.sampling_order == [[0, 1], [2], list(range(3, nb))]
    assert np.array_equal(got, want)


@pytest.mark.parametrize("C", [7, 130])
def test_ising_synchronous_sweep_with_clamped_block(device, C):
    n = 240
    rng, edges = _graph(n, 700, 3)
    b = rng.normal(0, 0.5, n).astype(np.float32)
    w = rng.normal(0, 0.5, len(edges)).astype(np.float32)
    blocks = _coloured_blocks(n, edges)
    free, clamped = blocks[:-1], blocks[-1:]
    off = [0, len(free)]
    log_case(f"ising one superblock over {len(free)} free blocks + clamped, C={C}")
    _, got, want = _ising_case(device, n, edges, b, w, 0.8, free, clamped, off, C, 3, 4, 44)
    assert np.array_equal(got, want)
    nf = sum(x.size for x in free)
    init = np.random.default_rng(4).integers(0, 2, (C, n)).astype(np.uint8)
    assert np.array_equal(got[:, nf:], init[:, nf:])


@pytest.mark.parametrize("C", [9, 200])
def test_ising_intra_block_edges_grouped(device, C):
    """Contiguous node ranges as blocks: edges run inside blocks too, so every
    block of a superblock (the last included) is staged."""
    n = 256
    rng, edges = _graph(n, 800, 5)
    b = rng.normal(0, 0.4, n).astype(np.float32)
    w = rng.normal(0, 0.4, len(edges)).astype(np.float32)
    blocks = [np.arange(i, i + 32, dtype=np.uint32) for i in range(0, n, 32)]
    off = [0, 3, 3, 4, 8]  # an empty superblock in the middle
    log_case(f"ising intra-block edges, superblocks={off}, C={C}")
    _, got, want = _ising_case(device, n, edges, b, w, 1.0, blocks, [], off, C, 3, 6, 55)
    assert np.array_equal(got, want)


def test_lattice_grouped_runs_on_csr(device):
    ebm, blocks = wl.lattice_ising(32, 0.2, 0.3, 0.1)
    blocks = [np.asarray(x.nodes if hasattr(x, "nodes") else x, np.uint32) for x in blocks]
    ungrouped = th.IsingSamplingProgram(ebm, blocks, [], device)
    assert ungrouped.kind == "lattice"
    ungrouped.close()
    edges = ebm.edges
    log_case("lattice 32^2 with both colours in one superblock")
    prog, got, want = _ising_case(device, ebm.n_nodes, edges, ebm.biases, ebm.weights, ebm.beta,
                                  blocks, [], [0, 2], 96, 5, 7, 66)
    assert prog.kind == "csr"
    assert np.array_equal(got, want)


def test_bipartite_grouped_runs_on_csr(device):
    V, H = 64, 128
    rng = np.random.default_rng(8)
    W = th.bf16_round(rng.normal(0, 0.2, (V, H)).astype(np.float32))[1]
    edges = np.array([(v, V + h) for v in range(V) for h in range(H)], np.uint32)
    b = rng.normal(0, 0.3, V + H).astype(np.float32)
    blocks = [np.arange(V, dtype=np.uint32), np.arange(V, V + H, dtype=np.uint32)]
    ebm = th.IsingEBM(V + H, edges, b, W.reshape(-1), 1.0)
    dense = th.IsingSamplingProgram(ebm, blocks, [], device, dense=True)
    assert dense.kind == "dense"
    dense.close()
    log_case("complete bipartite 64x128 with both sides in one superblock")
    prog, got, want = _ising_case(device, V + H, edges, b, W.reshape(-1), 1.0, blocks, [],
                                  [0, 2], 70, 3, 9, 77)
    assert prog.kind == "csr"
    assert np.array_equal(got, want)


@pytest.mark.parametrize("q,C,intra", [(3, 6, False), (4, 100, False), (5, 37, True),
                                         (24, 33, True), (40, 5, False)])
def test_categorical_grouped_blocks(device, q, C, intra):
    n = 180
    rng, edges = _graph(n, 500, 10 + q)
    W = rng.normal(0, 0.6, (len(edges), q, q)).astype(np.float32)
    bias = rng.normal(0, 0.5, (n, q)).astype(np.float32)
    if intra:
        blocks = [np.arange(i, i + 30, dtype=np.uint32) for i in range(0, n, 30)]
    else:
        blocks = _coloured_blocks(n, edges)
    free, clamped = blocks[:-1], blocks[-1:]
    nf = len(free)
    off = [0, 2, nf] if nf > 2 else [0, nf]
    log_case(f"categorical q={q} C={C} intra={intra} superblocks={off}")
    prog = th.CategoricalProgram(n, q, edges, W, bias, _nest(free, off), device,
                                 clamped_blocks=clamped)
    o = orc.Potts(n, q, edges, W, bias, free, clamped, superblocks=off)
    init = rng.integers(0, q, (C, prog.n_total)).astype(np.uint8)
    st = prog.new_state(C)
    st.set_global(init)
    th.run_blocks(th.RngKey(21), prog, st, (), 4)
    want, _ = o.run_blocks(21, init, 4)
    assert np.array_equal(st.get_global(), want)
    st.set_global(init)
    samples = th.sample_states(th.RngKey(22), prog, th.SamplingSchedule(2, 4, 3), st)
    assert np.array_equal(samples, o.sample_states(22, (2, 4, 3), init))
    st.close()


def test_moments_through_superblocks(device):
    n = 200
    rng, edges = _graph(n, 600, 23)
    b = rng.normal(0, 0.3, n).astype(np.float32)
    w = rng.normal(0, 0.4, len(edges)).astype(np.float32)
    blocks = _coloured_blocks(n, edges)
    off = [0, 2] + list(range(3, len(blocks) + 1))
    ebm = th.IsingEBM(n, edges, b, w, 0.9)
    prog = th.IsingSamplingProgram(ebm, _nest(blocks, off), [], device)
    o = orc.Ising(n, edges, b, w, 0.9, blocks, superblocks=off)
    C = 80
    init = rng.integers(0, 2, (C, n)).astype(np.uint8)
    nodes = rng.choice(n, 40, replace=False).astype(np.uint32)
    pairs = edges[rng.choice(len(edges), 60, replace=False)]
    log_case("estimate_moments through superblocks, C=80")
    st = prog.new_state(C)
    st.set_global(init)
    ns, es = th.estimate_moments(th.RngKey(24), nodes, pairs, prog, th.SamplingSchedule(3, 5, 2),
                                 st, return_sums=True)
    wns, wes, _, _ = o.estimate_moments(24, (3, 5, 2), init, nodes, pairs)
    assert np.array_equal(ns, wns)
    assert np.array_equal(es, wes)
    st.close()


def test_noalloc_on_grouped_program(device):
    n = 160
    rng, edges = _graph(n, 450, 25)
    b = rng.normal(0, 0.4, n).astype(np.float32)
    w = rng.normal(0, 0.5, len(edges)).astype(np.float32)
    blocks = _coloured_blocks(n, edges)
    off = [0, len(blocks)]
    ebm = th.IsingEBM(n, edges, b, w, 1.2)
    prog = th.IsingSamplingProgram(ebm, _nest(blocks, off), [], device)
    init = rng.integers(0, 2, (90, n)).astype(np.uint8)
    a, c = prog.new_state(90), prog.new_state(90)
    a.set_global(init)
    c.set_global(init)
    log_case("noalloc on a one-superblock program, C=90")
    _lib.check(_lib.load().thrml_run_blocks_noalloc(prog._h, 26, a._h, 5))
    th.run_blocks(th.RngKey(26), prog, c, (), 5)
    assert np.array_equal(a.get_global(), c.get_global())
    want, _ = orc.Ising(n, edges, b, w, 1.2, blocks, superblocks=off).run_blocks(26, init, 5)
    assert np.array_equal(a.get_global(), want)
    a.close()
    c.close()


@pytest.mark.parametrize("off,msg", [([1, 3], "start at 0"), ([0, 2], "end at the number"),
                                     ([0, 2, 1, 3], "must not decrease")])
def test_invalid_superblock_offsets(device, off, msg):
    n = 12
    edges = np.array([(0, 5), (1, 9), (4, 8)], np.uint32)
    blocks = [np.arange(0, 4, dtype=np.uint32), np.arange(4, 8, dtype=np.uint32),
              np.arange(8, 12, dtype=np.uint32)]
    ebm = th.IsingEBM(n, edges, np.zeros(n, np.float32), np.ones(3, np.float32), 1.0)
    fb, foff, fnodes = th._blocks_flat(blocks)
    sb = np.asarray(off, np.uint32)
    d = _lib.IsingDesc(n, 3, _lib.ptr(ebm.edge_u, _lib.ctypes.c_uint32),
                       _lib.ptr(ebm.edge_v, _lib.ctypes.c_uint32),
                       _lib.ptr(ebm.biases, _lib.ctypes.c_float),
                       _lib.ptr(ebm.weights, _lib.ctypes.c_float), 1.0, 3,
                       _lib.ptr(foff, _lib.ctypes.c_uint32), _lib.ptr(fnodes, _lib.ctypes.c_uint32),
                       0, None, None, 0, sb.size - 1, _lib.ptr(sb, _lib.ctypes.c_uint32))
    h = _lib.ctypes.c_void_p()
    with pytest.raises(th.ThrmlError, match=msg):
        _lib.check(_lib.load().thrml_ising_program_create(device.handle, _lib.ctypes.byref(d),
                                                           _lib.ctypes.byref(h)))
