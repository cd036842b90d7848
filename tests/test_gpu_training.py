"""GPU checks of estimate_kl_grad / IsingTrainingSpec
(crates/thrml-models/src/ising.rs:391-433,531-595), the main caller of the
sweep: a data-clamped positive phase and a free negative phase, each an
estimate_moments run, and grad = -beta (<.>_+ - <.>_-).

  - against the oracle: the same two moment runs (same keys, same data rows
    per chain) through the CPU restatement give identical f32 gradients;
  - against mathematics: on a 3 + 2 node RBM the sampled gradient matches the
    exact one, whose positive phase is E[s_h | v] = tanh(beta (b_h + sum_v J s_v))
    and whose negative phase is an enumeration of all 2^5 states.  A sign or
    phase-order mistake moves it by twice the gradient."""
import itertools

import numpy as np
import pytest

import pyoracle as orc
import thrml_hip as th
from conftest import log_case

pytestmark = pytest.mark.gpu


def _rbm_ebm(V, H, seed, scale):
    rng = np.random.default_rng(seed)
    edges = np.array([(v, V + h) for v in range(V) for h in range(H)], np.uint32)
    b = rng.normal(0, scale, V + H).astype(np.float32)
    w = rng.normal(0, scale, edges.shape[0]).astype(np.float32)
    return th.IsingEBM(V + H, edges, b, w, 0.9), edges, b, w


@pytest.mark.parametrize("C", [1, 3])
def test_kl_grad_matches_oracle(device, C):
    log_case(f"kl grad vs oracle C={C}")
    V, H = 6, 4
    ebm, edges, b, w = _rbm_ebm(V, H, 11 + C, 0.5)
    vis, hid = np.arange(V), np.arange(V, V + H)
    sp = th.SamplingSchedule(2, 5, 2)
    sn = th.SamplingSchedule(3, 4, 1)
    spec = th.IsingTrainingSpec(ebm, [th.Block(vis)], [], [th.Block(hid)],
                                [th.Block(vis), th.Block(hid)], sp, sn, device)
    rng = np.random.default_rng(C)
    data = rng.integers(0, 2, (8, V)).astype(np.float32)
    init_pos = [rng.integers(0, 2, (C, H)).astype(np.float32)]
    init_neg = [rng.integers(0, 2, (C, V)).astype(np.float32),
                rng.integers(0, 2, (C, H)).astype(np.float32)]
    nodes = np.arange(V + H)
    key = th.RngKey(2024 + C)
    gw, gb = th.estimate_kl_grad(key, spec, nodes, edges, [data], [], init_pos, init_neg)

    kp, kn = key.split_two()
    rows = [k.seed % data.shape[0] for k in kp.split(C)]
    o_pos = orc.Ising(V + H, edges, b, w, 0.9, [hid], [vis])
    st_pos = np.concatenate([init_pos[0], data[rows]], axis=1).astype(np.uint8)
    ns_p, es_p, _, _ = o_pos.estimate_moments(kp.seed, (2, 5, 2), st_pos, nodes, edges)
    o_neg = orc.Ising(V + H, edges, b, w, 0.9, [vis, hid], [])
    st_neg = np.concatenate(init_neg, axis=1).astype(np.uint8)
    ns_n, es_n, _, _ = o_neg.estimate_moments(kn.seed, (3, 4, 1), st_neg, nodes, edges)
    beta = np.float32(0.9)
    dp, dn = np.float32(C * 5), np.float32(C * 4)
    want_b = (ns_p.astype(np.float32) / dp - ns_n.astype(np.float32) / dn) * -beta
    want_w = (es_p.astype(np.float32) / dp - es_n.astype(np.float32) / dn) * -beta
    assert gb.dtype == np.float32 and gw.dtype == np.float32
    assert np.array_equal(gb, want_b)
    assert np.array_equal(gw, want_w)
    spec.close()


def test_kl_grad_matches_exact_enumeration(device):
    log_case("kl grad exact enumeration")
    V, H = 3, 2
    ebm, edges, b, w = _rbm_ebm(V, H, 5, 0.6)
    beta = 0.9
    vis, hid = np.arange(V), np.arange(V, V + H)
    data = np.array([[1, 0, 1]], np.float32)  # one row: every chain clamps it
    spec = th.IsingTrainingSpec(ebm, [th.Block(vis)], [], [th.Block(hid)],
                                [th.Block(vis), th.Block(hid)], th.SamplingSchedule(10, 40, 2),
                                th.SamplingSchedule(10, 40, 2), device)
    C = 4096
    rng = np.random.default_rng(0)
    init_pos = [rng.integers(0, 2, (C, H)).astype(np.float32)]
    init_neg = [rng.integers(0, 2, (C, V)).astype(np.float32),
                rng.integers(0, 2, (C, H)).astype(np.float32)]
    nodes = np.arange(V + H)
    gw, gb = th.estimate_kl_grad(th.RngKey(7), spec, nodes, edges, [data], [], init_pos, init_neg)

    # exact positive phase: visible spins fixed to the data, hidden independent
    sv = 2.0 * data[0] - 1.0
    J = w.reshape(V, H)
    mh = np.tanh(beta * (b[V:] + sv @ J))
    pos_b = np.concatenate([sv, mh])
    pos_w = (sv[:, None] * mh[None, :]).reshape(-1)
    # exact negative phase: all 2^5 states
    states = 2.0 * np.array(list(itertools.product([0, 1], repeat=V + H))) - 1.0
    E = -beta * (states @ b + (states[:, edges[:, 0]] * states[:, edges[:, 1]]) @ w)
    p = np.exp(-(E - E.min()))
    p /= p.sum()
    neg_b = p @ states
    neg_w = p @ (states[:, edges[:, 0]] * states[:, edges[:, 1]])
    want_b = -beta * (pos_b - neg_b)
    want_w = -beta * (pos_w - neg_w)
    print("grad_b", gb, "exact", want_b)
    print("grad_w", gw, "exact", want_w)
    assert np.abs(want_b).max() > 0.2  # the check has power against a sign mistake
    assert np.max(np.abs(gb - want_b)) < 0.02
    assert np.max(np.abs(gw - want_w)) < 0.02
    spec.close()
