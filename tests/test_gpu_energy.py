"""GPU per-chain energies (thrml_ising_energy, thrml_potts_energy) against the
oracle's energies (orc_ising_energy, orc_potts_energy, both f64 over the raw
edge lists; pinned on the CPU by the gamma / theta energy-difference
identities and the reference's own energy cases).

Tolerances.  The lattice, CSR and categorical kernels add the same f32 terms
as the oracle, in f64, in another order: |dE| <= 1e-9 * sum |term|.  The dense
kernel forms sum_v W[v][h] s_v on the matrix cores with f32 accumulation:
|dE| <= 1e-7 * sum |term|.  Cases: the reference's hand cases
(crates/thrml-models/tests/test_ising.rs:139-212), lattice and CSR programs
with clamped blocks and chain counts that are not multiples of 64, configs 2,
3 and 4 at full size, the dense program at config 5's shape, and the
categorical programs."""
import numpy as np
import pytest

import pyoracle as orc
import thrml_hip as th
from conftest import log_case
from thrml_hip import workloads as wl

pytestmark = pytest.mark.gpu


def _ising_scale(ebm):
    return abs(ebm.beta) * (np.abs(ebm.biases.astype(np.float64)).sum() +
                            np.abs(ebm.weights.astype(np.float64)).sum())


def _oracle(ebm, free, clamped=()):
    return orc.Ising(ebm.n_nodes, ebm.edges, ebm.biases, ebm.weights, ebm.beta,
                     [b.nodes if hasattr(b, "nodes") else b for b in free],
                     [b.nodes if hasattr(b, "nodes") else b for b in clamped])


def test_reference_cases(device):
    log_case("energy: reference hand cases")
    ebm = th.IsingEBM(3, [(0, 1), (1, 2)], [0.1, 0.2, 0.3], [0.5, -0.5], 1.0)
    prog = th.IsingSamplingProgram(ebm, [th.Block(np.arange(3))], [], device)
    st = prog.new_state(4)
    st.set_global(np.array([[0, 0, 0], [1, 1, 1], [1, 0, 1], [0, 1, 0]], np.uint8))
    assert np.allclose(th.ising_energy(prog, st), [0.6, -0.6, -0.2, 0.2], atol=1e-6)
    ebm = th.IsingEBM(4, [(0, 1), (1, 2), (2, 3)], np.zeros(4), np.ones(3), 1.0)
    prog = th.IsingSamplingProgram(ebm, [th.Block(np.arange(4))], [], device)
    st = prog.new_state(1)
    st.set_global(np.array([[1, 0, 1, 0]], np.uint8))
    assert np.allclose(th.ising_energy(prog, st), [3.0])


@pytest.mark.parametrize("L,C", [(32, 100), (10, 65), (64, 1)])
def test_lattice(device, L, C):
    log_case(f"energy: lattice L={L} C={C}")
    ebm, blocks = wl.lattice_ising(L, 0.3, 0.2, 0.5)
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    init = np.random.default_rng(L + C).integers(0, 2, (C, L * L)).astype(np.uint8)
    st = prog.new_state(C)
    st.set_global(init)
    got = th.ising_energy(prog, st)
    want = _oracle(ebm, blocks).energy(init)
    assert np.abs(got - want).max() <= 1e-9 * _ising_scale(ebm)
    # a fixed reduction order: the same state gives the same bits
    assert np.array_equal(got, th.ising_energy(prog, st))


@pytest.mark.parametrize("C", [1, 37, 130])
def test_csr_with_clamped_blocks(device, C):
    log_case(f"energy: csr clamped C={C}")
    rng = np.random.default_rng(C)
    n = 300
    perm = rng.permutation(n)
    free, clamped = [perm[:90], perm[90:170], perm[170:260]], [perm[260:]]
    edges = set()
    while len(edges) < 900:
        a, b = (int(x) for x in rng.integers(0, n, 2))
        if a != b:
            edges.add((a, b))
    edges = np.array(sorted(edges), np.uint32)
    ebm = th.IsingEBM(n, edges, rng.normal(0, 0.5, n), rng.normal(0, 0.6, len(edges)), 0.9)
    prog = th.IsingSamplingProgram(ebm, free, clamped, device)
    init = rng.integers(0, 2, (C, prog.n_total)).astype(np.uint8)
    st = prog.new_state(C)
    st.set_global(init)
    th.run_blocks(th.RngKey(5), prog, st, (), 3)
    state = st.get_global()
    want = _oracle(ebm, free, clamped).energy(state)
    assert np.abs(th.ising_energy(prog, st) - want).max() <= 1e-9 * _ising_scale(ebm)


def test_config2_full_size(device):
    log_case("energy: config 2 full size")
    ebm, blocks = wl.config_ising(2)
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    st = th.hinton_init(th.RngKey(5), prog, 64)
    th.run_blocks(th.RngKey(6), prog, st, (), 3)
    want = _oracle(ebm, blocks).energy(st.get_global())
    assert np.abs(th.ising_energy(prog, st) - want).max() <= 1e-9 * _ising_scale(ebm)


def test_config3_full_size(device):
    log_case("energy: config 3 full size")
    ebm, blocks = wl.config3()
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    st = th.hinton_init(th.RngKey(3), prog, 32)
    want = _oracle(ebm, blocks).energy(st.get_global())
    assert np.abs(th.ising_energy(prog, st) - want).max() <= 1e-9 * _ising_scale(ebm)


@pytest.mark.parametrize("V,H,C,nsel", [(1024, 4096, 4096, 6), (100, 300, 70, 70), (33, 17, 1, 1)])
def test_dense(device, V, H, C, nsel):
    log_case(f"energy: dense V={V} H={H} C={C}")
    rng = np.random.default_rng(V + H)
    if (V, H) == (1024, 4096):
        bits, Wf, bv, bh = wl.rbm(V, H, 0.01, 0.01)
        beta = 1.0
    else:
        bits, Wf = th.bf16_round(rng.normal(0, 0.2, (V, H)).astype(np.float32))
        bv = rng.normal(0, 0.3, V).astype(np.float32)
        bh = rng.normal(0, 0.3, H).astype(np.float32)
        beta = 0.7
    prog = th.RbmProgram(bits, bv, bh, beta, device)
    st = th.hinton_init(th.RngKey(9), prog, C)
    th.run_blocks(th.RngKey(10), prog, st, (), 2)
    got = th.ising_energy(prog, st)
    sel = np.linspace(0, C - 1, nsel).astype(int)
    edges = np.stack(np.meshgrid(np.arange(V), V + np.arange(H), indexing="ij"), -1).reshape(-1, 2)
    ebm = th.IsingEBM(V + H, edges, np.concatenate([bv, bh]), Wf.reshape(-1), beta)
    want = _oracle(ebm, [np.arange(V), V + np.arange(H)]).energy(st.get_global()[sel])
    assert np.abs(got[sel] - want).max() <= 1e-7 * _ising_scale(ebm)


def _potts_scale(W, bias):
    return np.abs(bias.astype(np.float64)).max(axis=-1).sum() + \
        np.abs(W.astype(np.float64)).reshape(len(W), -1).max(axis=-1).sum()


@pytest.mark.parametrize("L,q,C", [(16, 8, 40), (512, 8, 32)])
def test_potts_lattice(device, L, q, C):
    log_case(f"energy: potts lattice L={L} q={q} C={C}")
    n, edges, W, bias, blocks = wl.potts_lattice(L, q, 0.2, 0.1)
    prog = th.CategoricalProgram(n, q, edges, W, bias, blocks, device)
    init = np.random.default_rng(L).integers(0, q, (C, n)).astype(np.uint8)
    st = prog.new_state(C)
    st.set_global(init)
    th.run_blocks(th.RngKey(4), prog, st, (), 2)
    state = st.get_global()
    op = orc.Potts(n, q, edges, W, bias, [b.nodes for b in blocks])
    got = th.energy(prog, st)
    assert np.abs(got - op.energy(state)).max() <= 1e-9 * _potts_scale(W, bias)
    assert np.array_equal(got, th.potts_energy(prog, st))


@pytest.mark.parametrize("C", [1, 70])
def test_potts_random_graph(device, C):
    log_case(f"energy: potts random graph C={C}")
    rng = np.random.default_rng(C + 7)
    n, q = 200, 5
    edges = set()
    while len(edges) < 600:
        a, b = (int(x) for x in rng.integers(0, n, 2))
        if a != b:
            edges.add((a, b))
    edges = np.array(sorted(edges), np.uint32)
    W = rng.normal(0, 0.5, (len(edges), q, q)).astype(np.float32)
    bias = rng.normal(0, 0.3, (n, q)).astype(np.float32)
    perm = rng.permutation(n)
    blocks = [perm[:70], perm[70:140], perm[140:]]
    prog = th.CategoricalProgram(n, q, edges, W, bias, blocks, device)
    init = rng.integers(0, q, (C, n)).astype(np.uint8)
    st = prog.new_state(C)
    st.set_global(init)
    op = orc.Potts(n, q, edges, W, bias, blocks)
    assert np.abs(th.potts_energy(prog, st) - op.energy(init)).max() <= 1e-9 * _potts_scale(W, bias)


def test_energy_kind_errors(device):
    ebm, blocks = wl.lattice_ising(8, 0.1, 0.3, 0.05)
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    st = prog.new_state(3)
    with pytest.raises(th.ThrmlError, match="categorical"):
        th.potts_energy(prog, st)
    n, edges, W, bias, pblocks = wl.potts_lattice(8, 4, 0.5, 0.3)
    pprog = th.CategoricalProgram(n, 4, edges, W, bias, pblocks, device)
    pst = pprog.new_state(3)
    with pytest.raises(th.ThrmlError, match="spin program"):
        th.ising_energy(pprog, pst)
    with pytest.raises(th.ThrmlError, match="another program"):
        th.ising_energy(prog, pst)
