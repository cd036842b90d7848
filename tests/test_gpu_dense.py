"""GPU checks of the dense bipartite (RBM) sweep on the matrix cores.

The GPU accumulates sum_v W[v][h] (2 s_v - 1) in f32 in the MFMA order; the
oracle sums the exact products in double and rounds once, so decisions may
differ only where 2*gamma lies within 1e-5 of logit(u) (north_star's
threshold sites, counted and printed).  Cases: single half-sweeps of config 5
at its full shape (1024 x 4096, 4096 chains, every chain checked), a 1000 x
4000 model with 4000 chains (sites and chains past the ends of their tiles,
bf16 weights and f32 weights in three pieces), odd sizes that exercise the
padding, and the sampled moments of a tiny RBM against exact enumeration over
all 2^(V+H) states."""
import itertools

import numpy as np
import pytest

import pyoracle as orc
import thrml_hip as th
from conftest import log_case
from thrml_hip import workloads as wl

pytestmark = pytest.mark.gpu


def _check_half(prog, st, Wf, bv, bh, beta, blk, rng, sel):
    C = st.n_chains
    V, H = prog.V, prog.H
    g0 = st.get_global()
    key8 = rng.integers(0, 2**32, (C, 8), dtype=np.uint64).astype(np.uint32)
    prog.half_sweep(st, blk, key8)
    g1 = st.get_global()
    sv, sh = g0[sel, :V], g0[sel, V:]
    ov, oh, near = orc.rbm_half_sweep(Wf, bv, bh, beta, key8[sel], blk, sv, sh)
    got = g1[sel, :V] if blk == 0 else g1[sel, V:]
    want = ov if blk == 0 else oh
    other_got = g1[sel, V:] if blk == 0 else g1[sel, :V]
    other_want = sh if blk == 0 else sv
    assert np.array_equal(other_got, other_want), "the other block changed"
    diff = got != want
    assert not (diff & (near == 0)).any(), "decision differs away from the threshold"
    print(f"blk {blk}: {int(near.sum())} threshold sites, {int(diff.sum())} differ")
    return g1


@pytest.mark.parametrize("V,H,C,nsel,f32", [(1024, 4096, 4096, 4096, False),
                                            (1000, 4000, 4000, 4000, False),
                                            (1000, 4000, 4000, 4000, True),
                                            (100, 300, 70, 70, False),
                                            (256, 128, 200, 200, False), (33, 17, 1, 1, False),
                                            (300, 520, 300, 300, False)])
def test_half_sweep_parity(device, V, H, C, nsel, f32):
    log_case(f"dense half sweep V={V} H={H} C={C} f32={f32}")
    rng = np.random.default_rng(V + H + C)
    if (V, H) == (1024, 4096):
        bits, Wf, bv, bh = wl.rbm(V, H, 0.01, 0.01)
    else:
        Wf = rng.normal(0, 0.15 if V < 1000 else 0.02, (V, H)).astype(np.float32)
        if f32:
            bits = Wf  # held as three bf16 pieces
        else:
            bits, Wf = th.bf16_round(Wf)
        bv = rng.normal(0, 0.3, V).astype(np.float32)
        bh = rng.normal(0, 0.3, H).astype(np.float32)
    beta = 1.0 if V == 1024 else 0.8
    prog = th.RbmProgram(bits, bv, bh, beta, device)
    assert prog.kind == "dense" and prog.dense_pieces == (3 if f32 else 1)
    st = th.hinton_init(th.RngKey(3), prog, C)
    sel = np.sort(rng.choice(C, nsel, replace=False))
    _check_half(prog, st, Wf, bv, bh, beta, 1, rng, sel)
    _check_half(prog, st, Wf, bv, bh, beta, 0, rng, sel)


def _exact_ising_moments(n, edges, b, J, beta):
    states = np.array(list(itertools.product([0, 1], repeat=n)))
    t = 2 * states - 1
    E = -beta * (t @ b + (t[:, edges[:, 0]] * t[:, edges[:, 1]]) @ J)
    p = np.exp(-(E - E.min()))
    p /= p.sum()
    return p @ t, p @ (t[:, edges[:, 0]] * t[:, edges[:, 1]])


def test_tiny_rbm_moments_match_exact_enumeration(device):
    log_case("tiny rbm exact enumeration")
    V, H = 3, 4
    rng = np.random.default_rng(12)
    bits, Wf = th.bf16_round(rng.normal(0, 0.6, (V, H)).astype(np.float32))
    bv = rng.normal(0, 0.4, V).astype(np.float32)
    bh = rng.normal(0, 0.4, H).astype(np.float32)
    beta = 0.9
    prog = th.RbmProgram(bits, bv, bh, beta, device)
    edges = np.array([(v, V + h) for v in range(V) for h in range(H)], np.uint32)
    b = np.concatenate([bv, bh]).astype(np.float64)
    J = Wf.reshape(-1).astype(np.float64)
    m1, m2 = _exact_ising_moments(V + H, edges, b, J, beta)
    C = 4096
    st = th.hinton_init(th.RngKey(1), prog, C)
    th.run_blocks(th.RngKey(2), prog, st, (), 20)
    n_samples = 200
    nm, em = th.estimate_moments(th.RngKey(5), np.arange(V + H), edges, prog,
                                 th.SamplingSchedule(0, n_samples, 2), st)
    # chains are independent; consecutive samples of a chain are nearly so here
    se = np.sqrt(1.0 / (C * n_samples)) * 3.0
    assert np.max(np.abs(nm - m1)) < 6 * se, (nm, m1)
    assert np.max(np.abs(em - m2)) < 6 * se, (em, m2)


def test_dense_state_roundtrip_keeps_activations(device):
    """set_block rewrites the GEMM operands: a sweep after set_global equals one
    from the same state reached by hinton_init."""
    log_case("dense state roundtrip")
    rng = np.random.default_rng(0)
    bits, Wf = th.bf16_round(rng.normal(0, 0.2, (64, 96)).astype(np.float32))
    bv = rng.normal(0, 0.3, 64).astype(np.float32)
    bh = rng.normal(0, 0.3, 96).astype(np.float32)
    prog = th.RbmProgram(bits, bv, bh, 1.0, device)
    a = th.hinton_init(th.RngKey(7), prog, 130)
    init = a.get_global()
    b = prog.new_state(130)
    b.set_global(init)
    th.run_blocks(th.RngKey(9), prog, a, (), 3)
    th.run_blocks(th.RngKey(9), prog, b, (), 3)
    assert np.array_equal(a.get_global(), b.get_global())


def test_weight_pieces_found_on_the_device(device):
    """The fewest bf16 pieces that hold every weight exactly (one, two or
    three; the split and both weight layouts are made on the device), and the
    weights that have no exact three-piece form (not finite, or a nonzero
    piece below the normal bf16 range) are rejected."""
    log_case("dense weight pieces: 1, 2, 3 and rejections")
    rng = np.random.default_rng(5)
    V, H = 40, 70
    bv, bh = np.zeros(V, np.float32), np.zeros(H, np.float32)
    _, w1 = th.bf16_round(rng.normal(0, 0.3, (V, H)).astype(np.float32))
    w2 = w1.copy()
    w2[3, 5] = np.float32(1.0 + 2.0 ** -10)  # 1 + 2^-10: two pieces
    w3 = w1.copy()
    w3[7, 9] = np.float32(1.0 + 2.0 ** -10 + 2.0 ** -20)  # three pieces
    for w, want in ((w1, 1), (w2, 2), (w3, 3)):
        prog = th.RbmProgram(w, bv, bh, 1.0, device)
        assert prog.dense_pieces == want
    for bad in (np.inf, np.nan, np.float32(2.0 ** -130), np.float32(2.0 ** -118 * (1 + 2.0 ** -20))):
        w = w1.copy()
        w[1, 2] = bad
        with pytest.raises(th.ThrmlError, match="not a sum of three normal bf16 values"):
            th.RbmProgram(w, bv, bh, 1.0, device)
