"""Parity on the paths bench.py times, at their full shapes.

  - config 2 exactly as the bench runs it: 1024^2 torus, 64 chains, hinton
    init from RngKey(42).split_two(), a prebuilt MomentAccumulatorObserver
    over every node and edge writing device tensors, schedule (1, 24, 1):
    identical int64 sums and final state to the oracle's estimate_moments
    (crates/thrml-samplers/src/sampling.rs:178-320,
    crates/thrml-observers/src/moment.rs:157-237);
  - config 5 through thrml_run_blocks and the device key schedule: two
    sweeps of the 1024 x 4096 RBM with 4096 chains; every chain is replayed
    by the oracle's dense half-sweep with its block keys rebuilt from the
    reference's key tree (split(C)[c], split(n_iters)[s], split(2)[b],
    seed_from_u64); every chain without a threshold site must match exactly
    (sampling.rs:28-106); the same with arbitrary f32 weights (three bf16
    pieces per weight, crates/thrml-models/src/ising.rs:26-143 keeps its
    weights in f32);
  - categorical sample_states at config 4's full shape and on a small
    lattice with many observations, every observation against the oracle;
  - the moment counters' u32 -> u64 fold: saturated-bias programs (every
    spin pinned up) with chains x observations above 2^32, whose sums are
    exactly chains x observations, on the lattice kernel's fused counters
    and on the generic moment kernel;
  - the two discrete-factor programs the bench reports beside the
    configurations, at their full shapes and chain counts: config 4's Potts
    model written as categorical factors (d4) and the two-layer mixed
    spin / categorical torus (dmix), run_blocks against the oracle bit for
    bit (FactorSamplingProgram, crates/thrml-models/src/factor.rs:126-185);
  - the q = 32 Potts torus the bench reports as w32 (wide kernel):
    sample_states at every observation against the oracle."""
import numpy as np
import pytest

import pyoracle as orc
import thrml_hip as th
from conftest import log_case
from thrml_hip import workloads as wl

pytestmark = pytest.mark.gpu


def test_config2_bench_path_moments_and_state(device):
    import torch

    c = wl.CONFIGS[2]
    C = c["chains"]
    ebm, blocks = wl.config_ising(2)
    N = ebm.n_nodes
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    assert prog.kind == "lattice"
    sched = th.SamplingSchedule(1, 24, 1)
    observer = th.MomentAccumulatorObserver(
        prog, th.ising_moment_spec(np.arange(N, dtype=np.uint32), ebm.edges))
    out = (torch.empty(N, dtype=torch.int64, device="cuda"),
           torch.empty(ebm.edges.shape[0], dtype=torch.int64, device="cuda"))
    k_init, k_run = th.RngKey(c["key"]).split_two()
    log_case("config2 bench path: hinton + observer, schedule (1, 24, 1), 64 chains")
    st = th.hinton_init(k_init, prog, C)
    init = st.get_global()
    torch.cuda.synchronize()
    observer.sample_with_observation(k_run, sched, st, out=out)
    device.synchronize()
    ns, es = out[0].cpu().numpy(), out[1].cpu().numpy()
    final = st.get_global()
    o = orc.Ising(N, ebm.edges, ebm.biases, ebm.weights, ebm.beta, [b.nodes for b in blocks])
    assert np.array_equal(init, o.hinton_init(k_init.seed, C))
    wn, we, wst, near = o.estimate_moments(k_run.seed, (1, 24, 1), init,
                                           np.arange(N, dtype=np.uint32), ebm.edges)
    print(f"threshold sites in the oracle run: {near}")
    assert np.array_equal(final, wst)
    assert np.array_equal(ns, wn)
    assert np.array_equal(es, we)


def _chain_block_key8(root, C, chains, n_iters, n_blocks):
    """key8[s][b][k] of chain chains[k]: seed_from_u64 of
    split(split(split(root, C)[c], n_iters)[s], n_blocks)[b]."""
    ck = orc.rng_split(root, C)
    out = np.zeros((n_iters, n_blocks, len(chains), 8), np.uint32)
    for k, c in enumerate(chains):
        for s, sk in enumerate(orc.rng_split(ck[c], n_iters)):
            for b, bk in enumerate(orc.rng_split(sk, n_blocks)):
                out[s, b, k] = orc.seed_from_u64(bk)
    return out


def _config5_parity(device, weights, Wf, bv, bh, pieces, n_iters):
    c = wl.CONFIGS[5]
    C, V, H = c["chains"], c["V"], c["H"]
    prog = th.RbmProgram(weights, bv, bh, c["beta"], device)
    assert prog.dense_pieces == pieces
    st = th.hinton_init(th.RngKey(c["key"]), prog, C)
    init = st.get_global()
    log_case(f"config5 run_blocks, {pieces} weight piece(s), 4096 chains, {n_iters} sweeps")
    th.run_blocks(th.RngKey(7), prog, st, (), n_iters)
    got = st.get_global()
    sel = np.arange(C)  # every chain
    k8 = _chain_block_key8(7, C, sel, n_iters, 2)
    sv, sh = init[sel, :V].copy(), init[sel, V:].copy()
    dirty = np.zeros(len(sel), bool)
    for s in range(n_iters):
        sv, sh, nv = orc.rbm_half_sweep(Wf, bv, bh, c["beta"], k8[s, 0], 0, sv, sh)
        sv, sh, nh = orc.rbm_half_sweep(Wf, bv, bh, c["beta"], k8[s, 1], 1, sv, sh)
        dirty |= nv.any(axis=1) | nh.any(axis=1)
    want = np.concatenate([sv, sh], axis=1)
    same = (got[sel] == want).all(axis=1)
    print(f"{len(sel)} chains checked, {int(dirty.sum())} with threshold sites, "
          f"{int((~same).sum())} differ")
    assert same[~dirty].all(), "a chain without threshold sites differs"
    assert (~dirty).sum() >= 0.8 * len(sel)


def test_config5_run_blocks_through_key_schedule(device):
    c = wl.CONFIGS[5]
    bits, Wf, bv, bh = wl.rbm(c["V"], c["H"], c["w_std"], c["b_std"])
    _config5_parity(device, bits, Wf, bv, bh, 1, 2)


def test_config5_f32_weights(device):
    c = wl.CONFIGS[5]
    W, bv, bh = wl.rbm_f32(c["V"], c["H"], c["w_std"], c["b_std"])
    _config5_parity(device, W, W, bv, bh, 3, 1)


def _potts_sample_parity(device, n, q, edges, W, bias, blocks, C, sched, key, seed):
    prog = th.CategoricalProgram(n, q, edges, W, bias, blocks, device)
    init = np.random.default_rng(seed).integers(0, q, (C, n)).astype(np.uint8)
    st = prog.new_state(C)
    st.set_global(init)
    got = th.sample_states(th.RngKey(key), prog, th.SamplingSchedule(*sched), st)
    o = orc.Potts(n, q, edges, W, bias, [b.nodes if hasattr(b, "nodes") else b for b in blocks])
    want = o.sample_states(key, sched, init)
    assert got.shape == want.shape
    for k in range(got.shape[0]):
        assert np.array_equal(got[k], want[k]), f"observation {k} differs"


def test_categorical_sample_states_small_many_observations(device):
    log_case("categorical sample_states 16^2 q=4, schedule (2, 9, 3)")
    n, edges, W, bias, blocks = wl.potts_lattice(16, 4, 0.5, 0.3, cfg=9)
    _potts_sample_parity(device, n, 4, edges, W, bias, blocks, 40, (2, 9, 3), 5, 2)


def test_categorical_sample_states_config4_shape(device):
    c = wl.CONFIGS[4]
    log_case("categorical sample_states config 4 shape, schedule (1, 3, 1)")
    n, edges, W, bias, blocks = wl.potts_lattice(c["L"], c["q"], c["w_std"], c["b_std"])
    _potts_sample_parity(device, n, c["q"], edges, W, bias, blocks, c["chains"], (1, 3, 1),
                         c["key"], 4)


def _saturated_fold(device, ebm, blocks, C, n_samples, kind):
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    assert prog.kind == kind
    st = th.hinton_init(th.RngKey(1), prog, C)
    assert st.get_global().all()
    nodes = np.arange(ebm.n_nodes, dtype=np.uint32)
    ns, es = th.estimate_moments(th.RngKey(2), nodes, ebm.edges, prog,
                                 th.SamplingSchedule(1, n_samples, 1), st, return_sums=True)
    total = C * n_samples
    assert total > 2**32
    assert st.get_global().all()
    assert (ns == total).all() and (es == total).all()


def test_moment_fold_saturated_lattice(device):
    # 32^2 torus, bias 100 (every spin up), 65536 chains: the u32 counters
    # fold after 65535 observations; 65600 observations give 4.299e9 > 2^32
    log_case("moment fold: lattice 32^2, 65536 chains, 65600 observations")
    n, edges, up, lo = th.make_nearest_neighbor_lattice(32)
    ebm = th.IsingEBM(n, edges, np.full(n, 100.0, np.float32),
                      np.full(edges.shape[0], 0.3, np.float32))
    _saturated_fold(device, ebm, [up, lo], 65536, 65600, "lattice")


def test_moment_fold_saturated_csr(device):
    log_case("moment fold: CSR 6-node chain, 65536 chains, 65600 observations")
    edges = np.array([(i, i + 1) for i in range(5)], np.uint32)
    ebm = th.IsingEBM(6, edges, np.full(6, 100.0, np.float32), np.full(5, -0.7, np.float32))
    _saturated_fold(device, ebm, [th.Block([0, 2, 4]), th.Block([1, 3, 5])], 65536, 65600,
                    "csr")


def _factor_tuples(fs):
    out = []
    for f in fs:
        g = f.nodes.reshape(f.n_spin + f.n_cat, -1)
        out.append((list(g[:f.n_spin]), list(g[f.n_spin:]), f.weights, bool(f.flags & 1)))
    return out


def _discrete_bench_parity(device, n, kinds, q, fs, blocks, C, key, sweeps):
    prog = th.FactorSamplingProgram(kinds, q, fs, blocks, [], device)
    o = orc.Discrete(n, kinds, q, _factor_tuples(fs), [np.asarray(b) for b in blocks])
    rng = np.random.default_rng(key)
    kp = kinds[np.concatenate([np.asarray(b) for b in blocks])]
    init = np.where(kp[None] == 0, rng.integers(0, 2, (C, n)),
                    rng.integers(0, max(q, 2), (C, n))).astype(np.uint8)
    st = prog.new_state(C)
    st.set_global(init)
    th.run_blocks(th.RngKey(key), prog, st, (), sweeps)
    want, _ = o.run_blocks(key, init, sweeps)
    assert np.array_equal(st.get_global(), want)
    st.close()


def test_discrete_bench_d4_shape(device):
    c = wl.CONFIGS[4]
    log_case("discrete d4: config 4 Potts as factors, 32 chains, 2 sweeps")
    n, edges, W, bias, blocks = wl.potts_lattice(c["L"], c["q"], c["w_std"], c["b_std"])
    fs = [th.CategoricalEBMFactor([np.arange(n)], bias.reshape(n, c["q"], 1)),
          th.CategoricalEBMFactor([edges[:, 0], edges[:, 1]], W)]
    _discrete_bench_parity(device, n, np.ones(n, np.uint8), c["q"], fs,
                           [b.nodes for b in blocks], c["chains"], 61, 2)


def test_discrete_bench_dmix_shape(device):
    log_case("discrete dmix: two-layer 512^2 torus, q = 4, 32 chains, 2 sweeps")
    n, kinds, fs, blocks = wl.mixed_lattice(512, 4)
    _discrete_bench_parity(device, n, kinds, 4, fs, blocks, 32, 62, 2)


def test_wide_bench_w32_shape(device):
    # the bench's w32 workload: 256^2 torus Potts, q = 32, 32 chains, on the
    # wide kernel; run_blocks and sample_states against the oracle
    log_case("wide w32: 256^2 torus Potts q = 32, 32 chains, schedule (1, 2, 1)")
    n, edges, W, bias, blocks = wl.potts_lattice(256, 32, 0.2, 0.1)
    _potts_sample_parity(device, n, 32, edges, W, bias, blocks, 32, (1, 2, 1), 32, 33)
