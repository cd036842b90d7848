"""Categorical nodes with more than 16 categories (17..256, where the state
holds one byte per node; 257..65536 with two bytes is in test_gpu_potts.py and
test_gpu_discrete.py) on the device against the oracle, bit for bit: the wide
kernels (potts_wide_kernel, discrete_wide_kernel), whose lanes take one site
each and walk its categories one ChaCha8 block at a time
(CategoricalGibbsConditional, crates/thrml-samplers/src/softmax.rs:586-710;
categorical_sample, softmax.rs:60-97; word i*q + c of the block's stream).

  - CategoricalProgram on random graphs with edges inside blocks: q = 17, 18,
    20, 30, 32, 33, 64, 100, 256 (the row loads of q a multiple of 16, of 4,
    even q and odd q), run_blocks and energies; chain counts that are not
    multiples of 4;
  - sample_states at every observation (q = 24 lattice);
  - clamped blocks (q = 40); superblocks in test_gpu_superblocks.py;
  - the reference's strong-logit test at q = 40 without edges;
  - q = 65537 and q = 1 are rejected by CategoricalProgram, q = 65537 by
    FactorSamplingProgram.
The FactorSamplingProgram side (mixed models, Potts written as factors) is
in test_gpu_discrete.py."""
import numpy as np
import pytest

import pyoracle as orc
import thrml_hip as th
from conftest import log_case
from thrml_hip import workloads as wl

pytestmark = pytest.mark.gpu


def _random_potts(n, m, q, n_blocks, seed):
    rng = np.random.default_rng(seed)
    edges = set()
    while len(edges) < m:
        a, b = (int(v) for v in rng.integers(0, n, 2))
        if a != b:
            edges.add((a, b))
    edges = np.array(sorted(edges), np.uint32)
    W = rng.normal(0, 0.7, (len(edges), q, q)).astype(np.float32)
    bias = rng.normal(0, 0.5, (n, q)).astype(np.float32)
    perm = rng.permutation(n)
    cuts = np.sort(rng.choice(np.arange(1, n), n_blocks - 1, replace=False))
    return edges, W, bias, np.split(perm, cuts)


def _scale(W, bias):
    return np.abs(bias.astype(np.float64)).max(axis=-1).sum() + \
        np.abs(W.astype(np.float64)).reshape(len(W), -1).max(axis=-1).sum()


@pytest.mark.parametrize("q,C,m", [(17, 5, 300), (18, 7, 300), (20, 33, 300), (30, 40, 200),
                                   (32, 64, 300), (33, 3, 300), (64, 70, 200), (100, 9, 120),
                                   (256, 16, 60)])
def test_wide_random_program_parity(device, q, C, m):
    log_case(f"wide categorical random program q={q} C={C} edges={m}")
    n = 120
    edges, W, bias, blocks = _random_potts(n, m, q, 3, seed=q * 10 + C)
    prog = th.CategoricalProgram(n, q, edges, W, bias, blocks, device)
    init = np.random.default_rng(C).integers(0, q, (C, prog.n_total)).astype(np.uint8)
    st = prog.new_state(C)
    st.set_global(init)
    th.run_blocks(th.RngKey(3 * q + C), prog, st, (), 4)
    o = orc.Potts(n, q, edges, W, bias, blocks)
    want, near = o.run_blocks(3 * q + C, init, 4)
    print(f"near-tie sites in the oracle run: {near}")
    got = st.get_global()
    assert np.array_equal(got, want)
    assert got.max() < q
    assert np.abs(th.potts_energy(prog, st) - o.energy(want)).max() <= 1e-9 * _scale(W, bias)
    st.close()


def test_wide_lattice_sample_states(device):
    log_case("wide categorical sample_states 12^2 q=24, schedule (1, 4, 2)")
    q, C = 24, 37
    n, edges, W, bias, blocks = wl.potts_lattice(12, q, 0.5, 0.3, cfg=24)
    prog = th.CategoricalProgram(n, q, edges, W, bias, blocks, device)
    init = np.random.default_rng(24).integers(0, q, (C, n)).astype(np.uint8)
    st = prog.new_state(C)
    st.set_global(init)
    got = th.sample_states(th.RngKey(6), prog, th.SamplingSchedule(1, 4, 2), st)
    o = orc.Potts(n, q, edges, W, bias, [b.nodes for b in blocks])
    want = o.sample_states(6, (1, 4, 2), init)
    assert got.shape == want.shape
    for k in range(got.shape[0]):
        assert np.array_equal(got[k], want[k]), f"observation {k} differs"
    st.close()


def test_wide_clamped_blocks(device):
    log_case("wide categorical clamped blocks q=40")
    q, n, C = 40, 90, 21
    edges, W, bias, blocks = _random_potts(n, 200, q, 4, seed=40)
    free, clamped = blocks[:3], blocks[3:]
    prog = th.CategoricalProgram(n, q, edges, W, bias, free, device, clamped_blocks=clamped)
    init = np.random.default_rng(41).integers(0, q, (C, prog.n_total)).astype(np.uint8)
    st = prog.new_state(C)
    st.set_global(init)
    th.run_blocks(th.RngKey(9), prog, st, (), 3)
    want, _ = orc.Potts(n, q, edges, W, bias, free, clamped).run_blocks(9, init, 3)
    got = st.get_global()
    assert np.array_equal(got, want)
    nf = sum(len(b) for b in free)
    assert np.array_equal(got[:, nf:], init[:, nf:])
    st.close()


def test_wide_strong_logits_without_edges(device):
    # the reference's strong-logit test (softmax.rs:873-898) at q = 40 on a
    # program without edges (bias rows only): logit +30 at one category
    log_case("wide categorical strong logits q=40, no edges")
    q = 40
    bias = np.full((2, q), -30.0, np.float32)
    bias[0, 37] = 30.0
    bias[1, 21] = 30.0
    prog = th.CategoricalProgram(2, q, np.zeros((0, 2), np.uint32), np.zeros(0, np.float32), bias,
                                 [np.array([0, 1])], device)
    st = prog.new_state(300)
    th.run_blocks(th.RngKey(42), prog, st, (), 2)
    g = st.get_global()
    assert (g[:, 0] == 37).all() and (g[:, 1] == 21).all()
    st.close()


def test_q_range_checks(device):
    for q in (1, 65537):
        bias = np.zeros((2, q), np.float32)
        with pytest.raises(th.ThrmlError, match="q must lie in 2..65536"):
            th.CategoricalProgram(2, q, np.zeros((0, 2), np.uint32), np.zeros(0, np.float32), bias,
                                  [np.array([0, 1])], device)
    with pytest.raises(th.ThrmlError, match="q must lie in 2..65536"):
        th.FactorSamplingProgram(np.ones(2, np.uint8), 65537,
                                 [th.CategoricalEBMFactor([np.arange(2)],
                                                          np.zeros((2, 65537, 1), np.float32))],
                                 [np.array([0, 1])], [], device)
