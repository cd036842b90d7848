"""Clamped blocks on categorical and dense programs, and the dense path
behind IsingSamplingProgram (crates/thrml-core/src/blockspec.rs:15-67,
crates/thrml-models/src/factor.rs:152-185, crates/thrml-models/src/ising.rs:
342-433,531-595, crates/thrml-samplers/src/sampling.rs:81-106,178-320).

  - categorical programs with clamped blocks: run_blocks, sample_states and
    energies equal the oracle's; clamped values never change;
  - dense programs with a clamped side (the data-clamped positive phase):
    every chain replayed by the oracle's dense half-sweep on the reference
    key tree (one free block: the block key is the sweep key);
  - an IsingSamplingProgram on a complete bipartite edge list runs on the
    matrix cores (kind "dense") only when asked (dense=True), with bf16
    weights in one piece and any other f32 weights in three, and equals the
    oracle replay on every chain without a threshold site; by default it
    stays on the CSR kernel (the reference's slot order);
  - estimate_kl_grad on that RBM: both phases on the matrix cores; the
    gradient equals the one computed from the same runs' sample_states, and
    those trajectories equal the oracle replay on every chain without a
    threshold site (|2 gamma - logit u| < 1e-5);
  - the reference's training loop (crates/thrml-models/tests/
    test_train_mnist.rs:505-515: estimate_kl_grad, then an f32 SGD update of
    the weights and biases, then new programs) stays on the matrix cores
    through several updates, every trajectory replayed by the oracle."""
import numpy as np
import pytest

import pyoracle as orc
import thrml_hip as th
from conftest import log_case

pytestmark = pytest.mark.gpu


# ---------------------------------------------------------------------------
def _random_potts(n, m, q, seed):
    rng = np.random.default_rng(seed)
    edges = set()
    while len(edges) < m:
        a, b = (int(v) for v in rng.integers(0, n, 2))
        if a != b:
            edges.add((a, b))
    edges = np.array(sorted(edges), np.uint32)
    W = rng.normal(0, 0.7, (len(edges), q, q)).astype(np.float32)
    bias = rng.normal(0, 0.5, (n, q)).astype(np.float32)
    return rng, edges, W, bias


@pytest.mark.parametrize("q,C", [(3, 5), (8, 70), (4, 64)])
def test_potts_clamped_blocks_parity(device, q, C):
    log_case(f"categorical clamped blocks q={q} C={C}")
    n = 200
    rng, edges, W, bias = _random_potts(n, 600, q, 31 + q)
    perm = rng.permutation(n)
    free = [perm[:60], perm[60:120]]
    clamped = [perm[120:170], perm[170:]]
    prog = th.CategoricalProgram(n, q, edges, W, bias, free, device, clamped_blocks=clamped)
    assert prog.n_total == n
    o = orc.Potts(n, q, edges, W, bias, free, clamped)
    init = rng.integers(0, q, (C, n)).astype(np.uint8)
    st = prog.new_state(C)
    st.set_global(init)
    th.run_blocks(th.RngKey(9), prog, st, (), 7)
    got = st.get_global()
    want, _ = o.run_blocks(9, init, 7)
    assert np.array_equal(got, want)
    assert np.array_equal(got[:, 120:], init[:, 120:])
    e = th.potts_energy(prog, st)
    assert np.abs(e - o.energy(want)).max() < 1e-9 * (np.abs(W).sum() + np.abs(bias).sum())
    st.set_global(init)
    samples = th.sample_states(th.RngKey(10), prog, th.SamplingSchedule(2, 5, 2), st)
    wants = o.sample_states(10, (2, 5, 2), init)
    assert np.array_equal(samples, wants)


def test_potts_clamped_state_clamp_argument(device):
    """run_blocks with per-block arrays and state_clamp, as the reference
    calls it (sampling.rs:81-106): the clamp values are broadcast to every
    chain and the free blocks come back."""
    log_case("categorical run_blocks with state_clamp arrays")
    n, q = 40, 4
    rng, edges, W, bias = _random_potts(n, 90, q, 5)
    free, clamped = [np.arange(0, 15), np.arange(15, 30)], [np.arange(30, 40)]
    prog = th.CategoricalProgram(n, q, edges, W, bias, free, device, clamped_blocks=clamped)
    C = 6
    init = [rng.integers(0, q, (C, 15)).astype(np.float32) for _ in range(2)]
    clamp = [rng.integers(0, q, 10).astype(np.float32)]
    out = th.run_blocks(th.RngKey(4), prog, init, clamp, 5)
    full = np.concatenate([init[0], init[1], np.broadcast_to(clamp[0], (C, 10))], axis=1)
    want, _ = orc.Potts(n, q, edges, W, bias, free, clamped).run_blocks(4, full.astype(np.uint8), 5)
    assert np.array_equal(np.concatenate(out, axis=1), want[:, :30].astype(np.float32))


# ---------------------------------------------------------------------------
def _sweep_keys_run_blocks(root, C, n_iters, n_blocks):
    """k8[s][b][c]: seed_from_u64 of split(split(split(root, C)[c],
    n_iters)[s], n_blocks)[b] (sampling.rs:37,93)."""
    out = np.zeros((n_iters, n_blocks, C, 8), np.uint32)
    for c, ck in enumerate(orc.rng_split(root, C)):
        for s, sk in enumerate(orc.rng_split(ck, n_iters)):
            for b, bk in enumerate(orc.rng_split(sk, n_blocks)):
                out[s, b, c] = orc.seed_from_u64(bk)
    return out


def _sweep_keys_schedule(root, C, sched, n_blocks):
    """k8[s][b][c] of sample_with_observation's sweeps (sampling.rs:189-264):
    per chain (wk, sk) = split(key_c, 2); warm-up sweep w keyed by
    split(wk, n_warmup)[w]; sample i's step t by split(split(sk, n_samples -
    1)[i], steps)[t]; block keys split(sweep_key, n_blocks)."""
    n_warmup, n_samples, steps = sched
    n_sweeps = n_warmup + (n_samples - 1) * steps
    out = np.zeros((n_sweeps, n_blocks, C, 8), np.uint32)
    for c, ck in enumerate(orc.rng_split(root, C)):
        wk, sk = orc.rng_split(ck, 2)
        sweep = list(orc.rng_split(wk, n_warmup))
        for ks in orc.rng_split(sk, n_samples - 1):
            sweep += orc.rng_split(ks, steps)
        for s, key in enumerate(sweep):
            for b, bk in enumerate(orc.rng_split(key, n_blocks)):
                out[s, b, c] = orc.seed_from_u64(bk)
    return out


def _replay_dense(Wf, bv, bh, beta, k8, sides, sv, sh, observe_after=None):
    """Replays sweeps with the oracle's dense half-sweep: sweep s updates
    sides[b] with k8[s][b].  Returns (sv, sh, dirty chains, observations)."""
    dirty = np.zeros(sv.shape[0], bool)
    obs = []
    for s in range(k8.shape[0]):
        for b, side in enumerate(sides):
            sv, sh, near = orc.rbm_half_sweep(Wf, bv, bh, beta, k8[s, b], side, sv, sh)
            dirty |= near.any(axis=1)
        if observe_after is not None and s in observe_after:
            obs.append((sv.copy(), sh.copy()))
    return sv, sh, dirty, obs


def _rbm_model(V, H, seed, w_std=0.08, b_std=0.3):
    rng = np.random.default_rng(seed)
    bits, Wf = th.bf16_round(rng.normal(0, w_std, (V, H)).astype(np.float32))
    bv = rng.normal(0, b_std, V).astype(np.float32)
    bh = rng.normal(0, b_std, H).astype(np.float32)
    return rng, bits, Wf, bv, bh


def test_rbm_clamped_visible_run_blocks(device):
    log_case("dense program, visible clamped: 300 chains, 4 sweeps")
    V, H, C, beta = 160, 96, 300, 0.9
    rng, bits, Wf, bv, bh = _rbm_model(V, H, 41)
    prog = th.RbmProgram(bits, bv, bh, beta, device, clamped="visible")
    assert prog.kind == "dense"
    assert [len(b) for b in prog.free_blocks] == [H] and [len(b) for b in prog.clamped_blocks] == [V]
    data = rng.integers(0, 2, (C, V)).astype(np.uint8)
    h0 = rng.integers(0, 2, (C, H)).astype(np.uint8)
    st = prog.new_state(C)
    st.set_block(0, h0)
    st.set_block(1, data)
    th.run_blocks(th.RngKey(12), prog, st, (), 4)
    got_h, got_v = st.get_block(0), st.get_block(1)
    assert np.array_equal(got_v, data)
    k8 = _sweep_keys_run_blocks(12, C, 4, 1)
    _, sh, dirty, _ = _replay_dense(Wf, bv, bh, beta, k8, [1], data, h0)
    same = (got_h == sh).all(axis=1)
    print(f"{C} chains, {int(dirty.sum())} with threshold sites, {int((~same).sum())} differ")
    assert same[~dirty].all() and (~dirty).sum() >= 0.9 * C
    # the clamped side cannot be half-swept explicitly
    with pytest.raises(th.ThrmlError, match="clamped"):
        prog.half_sweep(st, 0, np.zeros((C, 8), np.uint32))


def test_rbm_clamped_hidden_run_blocks(device):
    log_case("dense program, hidden clamped: 70 chains, 3 sweeps")
    V, H, C, beta = 100, 260, 70, 1.0
    rng, bits, Wf, bv, bh = _rbm_model(V, H, 42)
    prog = th.RbmProgram(bits, bv, bh, beta, device, clamped="hidden")
    cond = rng.integers(0, 2, (C, H)).astype(np.uint8)
    v0 = rng.integers(0, 2, (C, V)).astype(np.uint8)
    st = prog.new_state(C)
    st.set_block(0, v0)
    st.set_block(1, cond)
    th.run_blocks(th.RngKey(13), prog, st, (), 3)
    k8 = _sweep_keys_run_blocks(13, C, 3, 1)
    sv, _, dirty, _ = _replay_dense(Wf, bv, bh, beta, k8, [0], v0, cond)
    same = (st.get_block(0) == sv).all(axis=1)
    assert same[~dirty].all() and (~dirty).sum() >= 0.9 * C
    assert np.array_equal(st.get_block(1), cond)


def _bipartite_ebm(V, H, Wf, bv, bh, beta, flip=False):
    vv, hh = np.meshgrid(np.arange(V), np.arange(V, V + H), indexing="ij")
    edges = np.stack([vv.ravel(), hh.ravel()], axis=1).astype(np.uint32)
    if flip:  # either orientation, any order
        edges = edges[:, ::-1].copy()
    return th.IsingEBM(V + H, edges, np.concatenate([bv, bh]), Wf.ravel(), beta)


def test_ising_program_complete_bipartite_routes_to_dense(device):
    log_case("IsingSamplingProgram on a complete bipartite graph: routing")
    V, H, C, beta = 128, 192, 256, 1.0
    rng, bits, Wf, bv, bh = _rbm_model(V, H, 43)
    ebm = _bipartite_ebm(V, H, Wf, bv, bh, beta)
    vis, hid = th.Block(np.arange(V)), th.Block(np.arange(V, V + H))
    prog = th.IsingSamplingProgram(ebm, [vis, hid], [], device, dense=True)
    assert prog.kind == "dense" and prog.dense_pieces == 1
    flipped = th.IsingSamplingProgram(_bipartite_ebm(V, H, Wf, bv, bh, beta, flip=True),
                                      [vis, hid], [], device, dense=True)
    assert flipped.kind == "dense"
    # the default keeps the reference's slot order
    assert th.IsingSamplingProgram(ebm, [vis, hid], [], device).kind == "csr"
    inexact = th.IsingEBM(V + H, ebm.edges, ebm.biases, ebm.weights + np.float32(1e-4), beta)
    p3 = th.IsingSamplingProgram(inexact, [vis, hid], [], device, dense=True)
    assert p3.kind == "dense" and p3.dense_pieces == 3
    # a weight with no exact three-piece form keeps the model on the CSR kernel
    w_sub = ebm.weights.copy()
    w_sub[17] = np.float32(2.0 ** -130)
    sub = th.IsingEBM(V + H, ebm.edges, ebm.biases, w_sub, beta)
    assert th.IsingSamplingProgram(sub, [vis, hid], [], device, dense=True).kind == "csr"
    small = _bipartite_ebm(32, 40, Wf[:32, :40], bv[:32], bh[:40], beta)
    assert th.IsingSamplingProgram(small, [np.arange(32), np.arange(32, 72)], [],
                                   device, dense=True).kind == "csr"
    # hidden block first: side 0 is then the hidden block (W transposed)
    swapped = th.IsingSamplingProgram(ebm, [hid, vis], [], device, dense=True)
    assert swapped.kind == "dense"
    st = th.hinton_init(th.RngKey(3), prog, C)
    init = st.get_global()
    o = orc.Ising(ebm.n_nodes, ebm.edges, ebm.biases, ebm.weights, beta,
                  [vis.nodes, hid.nodes])
    assert np.array_equal(init, o.hinton_init(3, C))
    th.run_blocks(th.RngKey(4), prog, st, (), 5)
    got = st.get_global()
    k8 = _sweep_keys_run_blocks(4, C, 5, 2)
    sv, sh, dirty, _ = _replay_dense(Wf, bv, bh, beta, k8, [0, 1], init[:, :V], init[:, V:])
    same = (got == np.concatenate([sv, sh], axis=1)).all(axis=1)
    print(f"{C} chains, {int(dirty.sum())} with threshold sites, {int((~same).sum())} differ")
    assert same[~dirty].all() and (~dirty).sum() >= 0.9 * C
    # the swapped program sweeps [hidden, visible]: replay with that order
    st2 = swapped.new_state(C)
    st2.set_block(0, init[:, V:])
    st2.set_block(1, init[:, :V])
    th.run_blocks(th.RngKey(4), swapped, st2, (), 3)
    k8 = _sweep_keys_run_blocks(4, C, 3, 2)
    sv2, sh2, dirty2, _ = _replay_dense(Wf, bv, bh, beta, k8, [1, 0], init[:, :V], init[:, V:])
    same2 = (st2.get_block(0) == sh2).all(axis=1) & (st2.get_block(1) == sv2).all(axis=1)
    assert same2[~dirty2].all() and (~dirty2).sum() >= 0.9 * C
    # energies of the routed program: the dense coupling term
    e = th.ising_energy(prog, st)
    assert np.abs(e - o.energy(got)).max() < 1e-6 * (np.abs(Wf).sum() + 1)


def _moment_sums(obs_v, obs_h, V, H):
    """Integer sums over chains and observations of t_i and t_v t_h (edge e =
    v H + h), t = 2s - 1."""
    ns = np.zeros(V + H, np.int64)
    es = np.zeros(V * H, np.int64)
    for sv, sh in zip(obs_v, obs_h):
        tv = 2 * sv.astype(np.int64) - 1
        th_ = 2 * sh.astype(np.int64) - 1
        ns[:V] += tv.sum(axis=0)
        ns[V:] += th_.sum(axis=0)
        es += (tv.T @ th_).ravel()
    return ns, es


def test_estimate_kl_grad_rbm_on_matrix_cores(device):
    log_case("estimate_kl_grad on an RBM through the dense path")
    V, H, C, beta = 128, 64, 192, 1.0
    rng, bits, Wf, bv, bh = _rbm_model(V, H, 44)
    ebm = _bipartite_ebm(V, H, Wf, bv, bh, beta)
    vis, hid = th.Block(np.arange(V)), th.Block(np.arange(V, V + H))
    sp, sn = (2, 4, 1), (3, 5, 2)
    spec = th.IsingTrainingSpec(ebm, [vis], [], [hid], [vis, hid], th.SamplingSchedule(*sp),
                                th.SamplingSchedule(*sn), device, dense=True)
    assert spec.program_positive.kind == "dense" and spec.program_negative.kind == "dense"
    batch = rng.integers(0, 2, (10, V)).astype(np.float32)
    hp0 = rng.integers(0, 2, (C, H)).astype(np.uint8)
    vn0 = rng.integers(0, 2, (C, V)).astype(np.uint8)
    hn0 = rng.integers(0, 2, (C, H)).astype(np.uint8)
    key = th.RngKey(2024)
    gw, gb = th.estimate_kl_grad(key, spec, np.arange(V + H), ebm.edges, [batch], [],
                                 [hp0.astype(np.float32)],
                                 [vn0.astype(np.float32), hn0.astype(np.float32)])
    key_pos, key_neg = key.split_two()
    rows = batch[[k.seed % batch.shape[0] for k in key_pos.split(C)]].astype(np.uint8)
    # the same runs' trajectories from sample_states (the same device path)
    pos = th.sample_states(key_pos, spec.program_positive, th.SamplingSchedule(*sp),
                           [hp0.astype(np.float32)], [rows.astype(np.float32)])
    neg = th.sample_states(key_neg, spec.program_negative, th.SamplingSchedule(*sn),
                           [vn0.astype(np.float32), hn0.astype(np.float32)])
    ns_p, es_p = _moment_sums([o[:, H:] for o in pos], [o[:, :H] for o in pos], V, H)
    ns_n, es_n = _moment_sums([o[:, :V] for o in neg], [o[:, V:] for o in neg], V, H)
    dp, dn = np.float32(C * sp[1]), np.float32(C * sn[1])
    want_w = (es_p.astype(np.float32) / dp - es_n.astype(np.float32) / dn) * -np.float32(beta)
    want_b = (ns_p.astype(np.float32) / dp - ns_n.astype(np.float32) / dn) * -np.float32(beta)
    assert np.array_equal(gw, want_w) and np.array_equal(gb, want_b)
    # the trajectories against the oracle replay on the reference key tree
    k8p = _sweep_keys_schedule(key_pos.seed, C, sp, 1)
    obs_p = [sp[0] - 1 + i * sp[2] for i in range(sp[1])]
    _, _, dirty_p, op = _replay_dense(Wf, bv, bh, beta, k8p, [1], rows, hp0, obs_p)
    k8n = _sweep_keys_schedule(key_neg.seed, C, sn, 2)
    obs_n = [sn[0] - 1 + i * sn[2] for i in range(sn[1])]
    _, _, dirty_n, on = _replay_dense(Wf, bv, bh, beta, k8n, [0, 1], vn0, hn0, obs_n)
    for k in range(sp[1]):
        same = (pos[k][:, :H] == op[k][1]).all(axis=1) & (pos[k][:, H:] == rows).all(axis=1)
        assert same[~dirty_p].all(), f"positive observation {k}"
    for k in range(sn[1]):
        same = (neg[k][:, :V] == on[k][0]).all(axis=1) & (neg[k][:, V:] == on[k][1]).all(axis=1)
        assert same[~dirty_n].all(), f"negative observation {k}"
    print(f"threshold chains: positive {int(dirty_p.sum())}, negative {int(dirty_n.sum())}")
    assert (~dirty_p).sum() >= 0.9 * C and (~dirty_n).sum() >= 0.9 * C
    spec.close()


def test_dense_f32_weights_in_three_pieces(device):
    log_case("IsingSamplingProgram dense=True, arbitrary f32 weights: 3 bf16 pieces")
    V, H, C, beta = 192, 320, 260, 0.9
    rng = np.random.default_rng(45)
    Wf = rng.normal(0, 0.09, (V, H)).astype(np.float32)  # not bf16-exact
    bv = rng.normal(0, 0.3, V).astype(np.float32)
    bh = rng.normal(0, 0.3, H).astype(np.float32)
    assert not np.array_equal(th.bf16_round(Wf)[1], Wf)
    ebm = _bipartite_ebm(V, H, Wf, bv, bh, beta)
    vis, hid = th.Block(np.arange(V)), th.Block(np.arange(V, V + H))
    prog = th.IsingSamplingProgram(ebm, [vis, hid], [], device, dense=True)
    assert prog.kind == "dense" and prog.dense_pieces == 3
    init = np.random.default_rng(46).integers(0, 2, (C, V + H)).astype(np.uint8)
    st = prog.new_state(C)
    st.set_global(init)
    th.run_blocks(th.RngKey(21), prog, st, (), 4)
    got = st.get_global()
    k8 = _sweep_keys_run_blocks(21, C, 4, 2)
    sv, sh, dirty, _ = _replay_dense(Wf, bv, bh, beta, k8, [0, 1], init[:, :V], init[:, V:])
    same = (got == np.concatenate([sv, sh], axis=1)).all(axis=1)
    print(f"{C} chains, {int(dirty.sum())} with threshold sites, {int((~same).sum())} differ")
    assert same[~dirty].all() and (~dirty).sum() >= 0.9 * C
    # the RbmProgram constructor takes f32 weights the same way
    rp = th.RbmProgram(Wf, bv, bh, beta, device)
    assert rp.kind == "dense" and rp.dense_pieces == 3
    st2 = rp.new_state(C)
    st2.set_global(init)
    th.run_blocks(th.RngKey(21), rp, st2, (), 4)
    assert np.array_equal(st2.get_global(), got)
    # the coupling term of the energy runs through the same pieces
    o = orc.Ising(ebm.n_nodes, ebm.edges, ebm.biases, ebm.weights, beta, [vis.nodes, hid.nodes])
    e = th.ising_energy(prog, st)
    assert np.abs(e - o.energy(got)).max() < 1e-6 * (np.abs(Wf).sum() + np.abs(bv).sum() +
                                                     np.abs(bh).sum())


def test_training_loop_stays_on_matrix_cores(device):
    """The reference's loop (test_train_mnist.rs:452-515): per batch, keys =
    key.split(3); hinton_init of both phases; estimate_kl_grad with keys[0];
    then weights += lr * grad_w and biases += lr * grad_b in f32 and new
    programs.  After the first update the weights are arbitrary f32 values:
    both programs stay on the matrix cores (three pieces), every trajectory
    equals the oracle's replay on each chain without a threshold site, and
    the gradient differs from the replay's by at most what the chains with
    threshold sites can move it."""
    V, H, C, beta = 256, 128, 256, 1.0
    rng = np.random.default_rng(47)
    Wf = th.bf16_round(rng.normal(0, 0.05, (V, H)).astype(np.float32))[1]  # bf16 at first
    b = rng.normal(0, 0.1, V + H).astype(np.float32)
    data = rng.integers(0, 2, (40, V)).astype(np.float32)
    vis, hid = th.Block(np.arange(V)), th.Block(np.arange(V, V + H))
    sp = sn = (4, 3, 2)
    lr = np.float32(0.01)
    key = th.RngKey(99)
    nodes = np.arange(V + H)
    for batch in range(3):
        log_case(f"dense training loop, batch {batch}")
        rows_b = data[batch * 10:(batch + 1) * 10]
        keys = key.split(3)
        key = keys[2]
        ebm = _bipartite_ebm(V, H, Wf, b[:V], b[V:], beta)
        spec = th.IsingTrainingSpec(ebm, [vis], [], [hid], [vis, hid], th.SamplingSchedule(*sp),
                                    th.SamplingSchedule(*sn), device, dense=True)
        pp, pn = spec.program_positive, spec.program_negative
        assert pp.kind == "dense" and pn.kind == "dense"
        assert pp.dense_pieces == pn.dense_pieces == (1 if batch == 0 else 3)
        hp0 = th.hinton_init(keys[0], pp, C).get_block(0)
        ng = th.hinton_init(keys[1], pn, C)
        vn0, hn0 = ng.get_block(0), ng.get_block(1)
        gw, gb = th.estimate_kl_grad(keys[0], spec, nodes, ebm.edges, [rows_b], [],
                                     [hp0.astype(np.float32)],
                                     [vn0.astype(np.float32), hn0.astype(np.float32)])
        key_pos, key_neg = keys[0].split_two()
        rows = rows_b[[k.seed % rows_b.shape[0] for k in key_pos.split(C)]].astype(np.uint8)
        k8p = _sweep_keys_schedule(key_pos.seed, C, sp, 1)
        obs_p = [sp[0] - 1 + i * sp[2] for i in range(sp[1])]
        _, _, dirty_p, op = _replay_dense(Wf, b[:V], b[V:], beta, k8p, [1], rows, hp0, obs_p)
        k8n = _sweep_keys_schedule(key_neg.seed, C, sn, 2)
        obs_n = [sn[0] - 1 + i * sn[2] for i in range(sn[1])]
        _, _, dirty_n, on = _replay_dense(Wf, b[:V], b[V:], beta, k8n, [0, 1], vn0, hn0, obs_n)
        pos = th.sample_states(key_pos, pp, th.SamplingSchedule(*sp), [hp0.astype(np.float32)],
                               [rows.astype(np.float32)])
        neg = th.sample_states(key_neg, pn, th.SamplingSchedule(*sn),
                               [vn0.astype(np.float32), hn0.astype(np.float32)])
        for k in range(sp[1]):
            same = (pos[k][:, :H] == op[k][1]).all(axis=1)
            assert same[~dirty_p].all(), f"batch {batch}: positive observation {k}"
        for k in range(sn[1]):
            same = (neg[k][:, :V] == on[k][0]).all(axis=1) & (neg[k][:, V:] == on[k][1]).all(axis=1)
            assert same[~dirty_n].all(), f"batch {batch}: negative observation {k}"
        # the replay's own gradient: moments differ only on chains with
        # threshold sites, each moving a mean by at most 2 / C per phase
        ns_p, es_p = _moment_sums([rows] * sp[1], [o[1] for o in op], V, H)
        ns_n, es_n = _moment_sums([o[0] for o in on], [o[1] for o in on], V, H)
        dp, dn = np.float32(C * sp[1]), np.float32(C * sn[1])
        ow = (es_p.astype(np.float32) / dp - es_n.astype(np.float32) / dn) * -np.float32(beta)
        ob = (ns_p.astype(np.float32) / dp - ns_n.astype(np.float32) / dn) * -np.float32(beta)
        bound = 2.0 * beta * (dirty_p.sum() + dirty_n.sum()) / C + 1e-6
        print(f"batch {batch}: threshold chains {int(dirty_p.sum())} + {int(dirty_n.sum())}, "
              f"grad diff {np.abs(gw - ow).max():.3g} / {np.abs(gb - ob).max():.3g} <= {bound:.3g}")
        assert np.abs(gw - ow).max() <= bound and np.abs(gb - ob).max() <= bound
        assert (~dirty_p).sum() >= 0.9 * C and (~dirty_n).sum() >= 0.9 * C
        # SGD in f32, as the reference does (test_train_mnist.rs:512-513)
        Wf = (Wf.ravel() + gw * lr).astype(np.float32).reshape(V, H)
        b = (b + gb * lr).astype(np.float32)
        spec.close()
    assert not np.array_equal(th.bf16_round(Wf)[1], Wf)


@pytest.mark.parametrize("V,H,C", [(100, 300, 300), (64, 1000, 70), (1024, 4096, 520)])
def test_dense_run_blocks_odd_shapes(device, V, H, C):
    """run_blocks of dense programs with sites past a multiple of 16 and of
    the 64-site tile, and chains past a multiple of 64 and of the 256-chain
    tile: every chain equals the oracle replay except at threshold sites."""
    log_case(f"dense run_blocks: V={V} H={H} C={C}")
    rng, bits, Wf, bv, bh = _rbm_model(V, H, 48 + V, w_std=0.08 if V < 1024 else 0.01)
    prog = th.RbmProgram(bits, bv, bh, 0.9, device)
    init = rng.integers(0, 2, (C, V + H)).astype(np.uint8)
    st = prog.new_state(C)
    st.set_global(init)
    th.run_blocks(th.RngKey(61), prog, st, (), 3)
    got = st.get_global()
    k8 = _sweep_keys_run_blocks(61, C, 3, 2)
    sv, sh, dirty, _ = _replay_dense(Wf, bv, bh, 0.9, k8, [0, 1], init[:, :V], init[:, V:])
    same = (got == np.concatenate([sv, sh], axis=1)).all(axis=1)
    print(f"{C} chains, {int(dirty.sum())} with threshold sites, {int((~same).sum())} differ")
    assert same[~dirty].all() and (~dirty).sum() >= 0.9 * C
