"""Benchmark of the block Gibbs sweep on one MI355X.

Default workload (the metric's own): 1024 x 1024
periodic Ising lattice, checkerboard 2-block Gibbs, biases ~N(0, 0.1),
couplings ~N(0.44, 0.05), beta = 1, 64 chains, 500 sweeps with magnetisation
and nearest-neighbour moments observed (schedule n_warmup=1, n_samples=500,
steps_per_sample=1).  One step = one sample_with_observation run of that
schedule through a MomentAccumulatorObserver built once for all nodes and all
edges, with the chains resident in HBM before the timed region starts and the
exact moment sums left in device memory (as the reference leaves its moments
in device tensors).

--workload c1 | c3 | c4 | c5 measures the other configurations the same way
(one step = run_blocks over the configuration's sweeps): c1 64^2 lattice with
256 chains and 1000 sweeps; c3 Erdos-Renyi 1M nodes, mean degree 12, greedy
colouring, 32 chains, 200 sweeps; c4 512^2 Potts q=8, 32 chains, 200 sweeps;
c5 dense 1024 x 4096 RBM (bf16 weights), 4096 chains, 200 sweeps.

metric: node-updates/s = chains * nodes * sweeps / time.
roofline: the workload's sweep kernel.  Algorithmic bytes per sweep (int8-
  equivalent state read + written once per chain, parameters once):
  lattice 2CN + 4N + 4E, irregular 2CN + 4N + 16E, Potts 2CN + 4qN + 4q^2E;
  dense: 4CVH flops per sweep against the bf16 matrix-core peak.  Divided by
  the kernel time from HIP events recorded on the library stream.
  traffic: HBM bytes per launch from the committed rocprofv3 counter summary.
valu_roofline: the same launch against the vector-ALU issue peak (614.4 G
  wave-instructions/s), from the committed SQ_INSTS_VALU counts per launch.
cpu_baseline: the CPU oracle (a C restatement of the reference's sweep),
  OpenMP over chains (one thread per chain, the box's CPU share of 16
  threads), on a bounded sample of the same program; with the host's nproc
  and CPU model, and (c2) a single-thread row in the reference's op-by-op
  order (op_by_op_1_thread).
configs: the default run also measures every other configuration the same
  way (CONFIG_STEPS steps each after one warm-up step): value, ms_per_step,
  roofline and valu_roofline per configuration (--no-configs skips them).
--energy N: also times N per-chain energy evaluations of the workload's state
  (energy_ms_per_call; outside the timed sweep region).
widened: the default run also measures two programs over general discrete
  factors (FactorSamplingProgram, the general discrete kernel): d4, config 4's
  Potts model written as categorical factors, and dmix, a two-layer spin /
  categorical torus (--workload d4 | dmix makes either the headline), then
  w32, a q = 32 Potts torus on the wide categorical kernel, and c5f32,
  config 5's RBM with f32 weights (three bf16 pieces per weight).
parity: with the CPU leg (not --no-cpu), every configuration and widened
  row also carries an untimed parity replay: a few sweeps of its program on
  the GPU from a fixed state and key against the oracle's (config 1: the
  configuration's whole 1000-sweep run; config 2: its observer path with all
  moments), with the number of site updates within 1e-5 of their threshold
  and, for the dense path, the chains that differ without one.
--gemm-reference (c5): also times the vendor bf16 GEMM (torch.matmul, which
  calls hipBLASLt) on the two half-sweep shapes, without any sampling, as a
  reference point for the matrix-core fraction these shapes allow.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "thrml-rs_amd"))

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0


VALU_PEAK_GWIS = 614.4  # 256 CUs x 1 wave-instruction per clock x 2.4 GHz


def _profile_value(name, key):
    """A `key: value` figure from the committed rocprofv3 summary
    profiles/<name>, if present."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith(key + ":"):
                return float(line.split(":", 1)[1])
    return None


def _traffic_from_profiles(name):
    """HBM bytes per launch (FETCH_SIZE + WRITE_SIZE, calibrated)."""
    return _profile_value(name, "traffic_bytes_per_launch")


def _oracle():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as orc

    return orc


def _timed(fn, reps):
    t0 = time.perf_counter()
    for i in range(reps):
        fn(i)
    return time.perf_counter() - t0


def _n_keys(args):
    """Run keys a workload prepares: enough for the timed, warm-up and
    event-timed steps of the headline and of the `configs` measurements."""
    return 256 + args.warmup + args.steps


def _scaled_sample(run, target_s, first=1):
    """Times run(n) for a first small n, then for n scaled to ~target_s."""
    dt = _timed(lambda i: run(first), 1)
    n = max(first, int(first * target_s / max(dt, 1e-3)))
    return n, _timed(lambda i: run(n), 1)


# ---------------------------------------------------------------------------
def cpu_ising(ebm, blocks, target_s, moments):
    import numpy as np

    orc = _oracle()
    o = orc.Ising(ebm.n_nodes, ebm.edges, ebm.biases, ebm.weights, ebm.beta,
                  [b.nodes for b in blocks])
    threads = orc.threads()
    n = ebm.n_nodes
    init = np.zeros((threads, n), np.uint8)
    if moments:
        nodes = np.arange(n, dtype=np.uint32)
        sweeps, dt = _scaled_sample(
            lambda k: o.estimate_moments(7, (1, k, 1), init, nodes, ebm.edges, threads),
            target_s, 2)
        what = f"schedule (1, {sweeps}, 1) with all node and edge moments"
    else:
        sweeps, dt = _scaled_sample(lambda k: o.run_blocks(7, init, k, threads), target_s, 1)
        what = f"run_blocks, {sweeps} sweeps"
    return {"value": threads * n * sweeps / dt, "unit": "node-updates/s", "cores": threads,
            "kind": "port",
            "sample": f"oracle on the same program: {threads} chains (one per thread), {what} "
                      f"({dt:.1f} s)"}


def cpu_potts(n, q, edges, W, bias, blocks, target_s):
    import numpy as np

    orc = _oracle()
    o = orc.Potts(n, q, edges, W, bias, [b.nodes for b in blocks])
    threads = orc.threads()
    init = np.zeros((threads, n), np.uint8)
    sweeps, dt = _scaled_sample(lambda k: o.run_blocks(7, init, k, threads), target_s, 1)
    return {"value": threads * n * sweeps / dt, "unit": "node-updates/s", "cores": threads,
            "kind": "port",
            "sample": f"oracle run_blocks on the same program: {threads} chains (one per thread) "
                      f"x {sweeps} sweeps ({dt:.1f} s)"}


def cpu_rbm(Wf, bv, bh, beta, target_s):
    import numpy as np

    orc = _oracle()
    threads = orc.threads()
    V, H = Wf.shape
    rng = np.random.default_rng(0)

    def run(chains):
        sv = np.zeros((chains, V), np.uint8)
        sh = np.zeros((chains, H), np.uint8)
        k8 = rng.integers(0, 2**32, (chains, 8), dtype=np.uint64).astype(np.uint32)
        sv, sh, _ = orc.rbm_half_sweep(Wf, bv, bh, beta, k8, 1, sv, sh, n_threads=threads)
        orc.rbm_half_sweep(Wf, bv, bh, beta, k8, 0, sv, sh, n_threads=threads)

    chains, dt = _scaled_sample(run, target_s, threads)
    return {"value": chains * (V + H) / dt, "unit": "node-updates/s", "cores": threads,
            "kind": "port",
            "sample": f"oracle dense half-sweeps (double accumulation) on the same 1024 x 4096 "
                      f"model: {chains} chains x 1 sweep ({dt:.1f} s)"}


def cpu_discrete(n, kinds, q, factors, blocks, target_s):
    import numpy as np

    orc = _oracle()
    fs = []
    for f in factors:
        g = f.nodes.reshape(f.n_spin + f.n_cat, -1)
        fs.append((list(g[:f.n_spin]), list(g[f.n_spin:]), f.weights, bool(f.flags & 1)))
    o = orc.Discrete(n, kinds, q, fs, [np.asarray(b) for b in blocks])
    threads = orc.threads()
    init = np.zeros((threads, n), np.uint8)
    sweeps, dt = _scaled_sample(lambda k: o.run_blocks(7, init, k, threads), target_s, 1)
    return {"value": threads * n * sweeps / dt, "unit": "node-updates/s", "cores": threads,
            "kind": "port",
            "sample": f"oracle run_blocks on the same program: {threads} chains (one per thread) "
                      f"x {sweeps} sweeps ({dt:.1f} s)"}


# ---------------------------------------------------------------------------
# Parity replay (part of the CPU leg, untimed): the workload's program runs a
# few sweeps on the GPU from a fixed state and key, the oracle runs the same
# sweeps, and the line reports whether the states agree and how many site
# updates fell within 1e-5 of their sampling threshold (|2 gamma - logit u|,
# or the top two Gumbel scores), where the reference's own f32 rounding could
# decide either way.
def _parity_record(got, want, near, sweeps, C, what, dirty=None):
    import numpy as np

    diff = (got != want).any(axis=1)
    rec = {"sweeps": sweeps, "chains": C, "chains_checked": int(got.shape[0]),
           "identical": bool(not diff.any()), "differing_chains": int(diff.sum()),
           "threshold_sites": int(near), "replay": what}
    if dirty is not None:
        rec["chains_with_threshold_sites"] = int(dirty.sum())
        rec["differing_chains_without_threshold_site"] = int((diff & ~dirty).sum())
        rec["identical_except_threshold_sites"] = bool(not (diff & ~dirty).any())
    return rec


def parity_spin(th, prog, ebm, blocks, init, key, sweeps):
    """run_blocks of a lattice or CSR Ising program against the oracle."""
    orc = _oracle()
    C = init.shape[0]
    st = prog.new_state(C)
    st.set_global(init)
    th.run_blocks(th.RngKey(key), prog, st, (), sweeps)
    got = st.get_global()
    st.close()
    o = orc.Ising(ebm.n_nodes, ebm.edges, ebm.biases, ebm.weights, ebm.beta,
                  [b.nodes for b in blocks])
    want, near = o.run_blocks(key, init, sweeps)
    return _parity_record(got, want, near, sweeps, C,
                          f"run_blocks(RngKey({key}), {sweeps} sweeps), every chain, oracle")


def parity_moments(th, prog, ebm, blocks, init, key, sweeps):
    """Config 2's observer path (schedule (1, sweeps, 1), every node and edge
    moment) against the oracle's estimate_moments: final state and int64 sums."""
    import numpy as np

    orc = _oracle()
    C, N = init.shape
    st = prog.new_state(C)
    st.set_global(init)
    nodes = np.arange(N, dtype=np.uint32)
    ns, es = th.estimate_moments(th.RngKey(key), nodes, ebm.edges, prog,
                                 th.SamplingSchedule(1, sweeps, 1), st, return_sums=True)
    got = st.get_global()
    st.close()
    o = orc.Ising(N, ebm.edges, ebm.biases, ebm.weights, ebm.beta, [b.nodes for b in blocks])
    wn, we, want, near = o.estimate_moments(key, (1, sweeps, 1), init, nodes, ebm.edges)
    rec = _parity_record(got, want, near, sweeps, C,
                         f"estimate_moments(RngKey({key}), schedule (1, {sweeps}, 1)), all node "
                         f"and edge moments, every chain, oracle")
    rec["moment_sums_identical"] = bool(np.array_equal(ns, wn) and np.array_equal(es, we))
    rec["identical"] = rec["identical"] and rec["moment_sums_identical"]
    return rec


def parity_potts(th, prog, n, q, edges, W, bias, blocks, init, key, sweeps):
    orc = _oracle()
    C = init.shape[0]
    st = prog.new_state(C)
    st.set_global(init)
    th.run_blocks(th.RngKey(key), prog, st, (), sweeps)
    got = st.get_global()
    st.close()
    o = orc.Potts(n, q, edges, W, bias, [b.nodes for b in blocks])
    want, near = o.run_blocks(key, init, sweeps)
    return _parity_record(got, want, near, sweeps, C,
                          f"run_blocks(RngKey({key}), {sweeps} sweeps), every chain, oracle")


def parity_discrete(th, prog, n, kinds, q, factors, blocks, init, key, sweeps):
    import numpy as np

    orc = _oracle()
    C = init.shape[0]
    st = prog.new_state(C)
    st.set_global(init)
    th.run_blocks(th.RngKey(key), prog, st, (), sweeps)
    got = st.get_global()
    st.close()
    fs = []
    for f in factors:
        g = f.nodes.reshape(f.n_spin + f.n_cat, -1)
        fs.append((list(g[:f.n_spin]), list(g[f.n_spin:]), f.weights, bool(f.flags & 1)))
    o = orc.Discrete(n, kinds, q, fs, [np.asarray(b) for b in blocks])
    want, near = o.run_blocks(key, init, sweeps)
    return _parity_record(got, want, near, sweeps, C,
                          f"run_blocks(RngKey({key}), {sweeps} sweeps), every chain, oracle")


def parity_dense(th, prog, Wf, bv, bh, beta, init, key, sweeps):
    """run_blocks of the dense program against the oracle's dense half-sweeps
    (exact products summed in double) with every chain's block keys rebuilt
    from the reference's key tree: split(C)[c], split(sweeps)[s], split(2)[b],
    seed_from_u64.  The matrix cores sum in another order than the reference's
    slot order, so decisions may differ at threshold sites only."""
    import numpy as np

    orc = _oracle()
    C = init.shape[0]
    V = Wf.shape[0]
    st = prog.new_state(C)
    st.set_global(init)
    th.run_blocks(th.RngKey(key), prog, st, (), sweeps)
    got = st.get_global()
    st.close()
    k8 = np.zeros((sweeps, 2, C, 8), np.uint32)
    for c, ck in enumerate(orc.rng_split(key, C)):
        for s, sk in enumerate(orc.rng_split(ck, sweeps)):
            for b, bk in enumerate(orc.rng_split(sk, 2)):
                k8[s, b, c] = orc.seed_from_u64(bk)
    sv, sh = init[:, :V].copy(), init[:, V:].copy()
    dirty = np.zeros(C, bool)
    near = 0
    for s in range(sweeps):
        sv, sh, nv = orc.rbm_half_sweep(Wf, bv, bh, beta, k8[s, 0], 0, sv, sh)
        sv, sh, nh = orc.rbm_half_sweep(Wf, bv, bh, beta, k8[s, 1], 1, sv, sh)
        dirty |= nv.any(axis=1) | nh.any(axis=1)
        near += int(nv.sum()) + int(nh.sum())
    want = np.concatenate([sv, sh], axis=1)
    return _parity_record(got, want, near, sweeps, C,
                          f"run_blocks(RngKey({key}), {sweeps} sweep(s)), every chain, oracle "
                          f"dense half-sweeps on the reference key tree", dirty)


def _random_state(C, n, q, seed, kinds=None):
    """A seeded random global state: categories 0..q-1, or 0/1 where kinds
    marks a spin node (kinds[i] == 0)."""
    import numpy as np

    x = np.random.default_rng(seed).integers(0, q, (C, n)).astype(np.uint8)
    if kinds is not None:
        x = np.where(np.asarray(kinds)[None, :] == 0, x & 1, x).astype(np.uint8)
    return x


# ---------------------------------------------------------------------------
def kernel_time(dev, fn, reps=2):
    """Average launch duration (ms) of the sweep kernels over reps calls of fn:
    HIP events on the library stream, one before the first launch and one
    after the last, over the launch count (an event pair around every launch
    would add the markers' own microseconds to each)."""
    dev.enable_timing(True, span=True)
    for i in range(reps):
        fn(i)
    dev.synchronize()
    ms, n = dev.kernel_time(0)
    dev.enable_timing(False)
    return ms, n


def workload_c2(args, th, wl, torch):
    import numpy as np

    c = wl.CONFIGS[2]
    C, sweeps = c["chains"], c["sweeps"]
    ebm, blocks = wl.config_ising(2)
    N, E = ebm.n_nodes, ebm.edge_u.size
    dev = th.Device(0)
    prog = th.IsingSamplingProgram(ebm, blocks, [], dev)
    assert prog.kind == "lattice"
    sched = th.SamplingSchedule(1, sweeps, 1)
    observer = th.MomentAccumulatorObserver(
        prog, th.ising_moment_spec(np.arange(N, dtype=np.uint32), ebm.edges))
    out = (torch.empty(N, dtype=torch.int64, device="cuda"),
           torch.empty(E, dtype=torch.int64, device="cuda"))
    k_init, k_run = th.RngKey(c["key"]).split_two()
    st = th.hinton_init(k_init, prog, C)
    keys = k_run.split(_n_keys(args))
    torch.cuda.synchronize()
    dev.synchronize()

    def step(i):
        observer.sample_with_observation(keys[i], sched, st, out=out)

    res = {"config": {"workload": "ising_lattice_1024_c64_500sweeps_moments", "L": 1024,
                      "chains": C, "sweeps_per_step": sweeps, "blocks": 2,
                      "schedule": [1, sweeps, 1], "moments": "all nodes + all edges"},
           "dtype": "f32"}
    return dev, step, C * N * sweeps, res, dict(
        kernel="lattice_half_kernel", bytes_per_launch=(2 * C * N + 4 * N + 4 * E) / 2.0,
        traffic="lattice_half_kernel_c2_traffic.txt", valu="lattice_half_kernel_c2_valu.txt",
        timing_step=lambda i: step(-1 - i),
        extra=lambda: {"sweep_only_node_updates_per_s": _sweep_only(th, dev, prog, st, C * N,
                                                                   sweeps)},
        energy=lambda: th.ising_energy(prog, st),
        cpu=lambda: cpu_ising(ebm, blocks, args.cpu_seconds, True),
        opbyop=lambda: cpu_opbyop(ebm, blocks, args.cpu_seconds / 2),
        parity=lambda: parity_moments(th, prog, ebm, blocks, th.hinton_init(k_init, prog, C)
                                      .get_global(), k_run.seed, 8))


def _sweep_only(th, dev, prog, st, per_sweep, sweeps):
    t0 = time.perf_counter()
    th.run_blocks(th.RngKey(99), prog, st, (), sweeps)
    dev.synchronize()
    return per_sweep * sweeps / (time.perf_counter() - t0)


def _run_blocks_workload(th, dev, prog, st, sweeps, keys):
    def step(i):
        th.run_blocks(keys[i], prog, st, (), sweeps)
    return step


def workload_c1(args, th, wl, torch):
    c = wl.CONFIGS[1]
    C, sweeps = c["chains"], c["sweeps"]
    ebm, blocks = wl.config_ising(1)
    N, E = ebm.n_nodes, ebm.edge_u.size
    dev = th.Device(0)
    prog = th.IsingSamplingProgram(ebm, blocks, [], dev)
    k_init, k_run = th.RngKey(c["key"]).split_two()
    st = th.hinton_init(k_init, prog, C)
    keys = k_run.split(_n_keys(args))
    step = _run_blocks_workload(th, dev, prog, st, sweeps, keys)
    res = {"config": {"workload": "ising_lattice_64_c256_1000sweeps", "L": 64, "chains": C,
                      "sweeps_per_step": sweeps, "blocks": 2}, "dtype": "f32"}
    return dev, step, C * N * sweeps, res, dict(
        kernel="lattice_half_kernel", bytes_per_launch=(2 * C * N + 4 * N + 4 * E) / 2.0,
        traffic="lattice_half_kernel_c1_traffic.txt", valu="lattice_half_kernel_c1_valu.txt",
        timing_step=lambda i: step(-1 - i), extra=lambda: {},
        energy=lambda: th.ising_energy(prog, st),
        cpu=lambda: cpu_ising(ebm, blocks, args.cpu_seconds, False),
        # the configuration's whole run: hinton init, then 1000 sweeps
        parity=lambda: parity_spin(th, prog, ebm, blocks, th.hinton_init(k_init, prog, C)
                                   .get_global(), keys[0].seed, sweeps))


def workload_c3(args, th, wl, torch):
    c = wl.CONFIGS[3]
    C, sweeps = c["chains"], c["sweeps"]
    t0 = time.perf_counter()
    ebm, blocks = wl.config3()
    dev = th.Device(0)
    prog = th.IsingSamplingProgram(ebm, blocks, [], dev)
    build_s = time.perf_counter() - t0
    N, E = ebm.n_nodes, ebm.edge_u.size
    st = th.hinton_init(th.RngKey(c["key"]), prog, C)
    keys = th.RngKey(c["key"] + 1).split(_n_keys(args))
    step = _run_blocks_workload(th, dev, prog, st, sweeps, keys)
    K = len(blocks)
    res = {"config": {"workload": "ising_er_1m_deg12_c32_200sweeps", "nodes": N, "edges": E,
                      "colour_blocks": K, "chains": C, "sweeps_per_step": sweeps,
                      "program_build_s": build_s}, "dtype": "f32"}
    return dev, step, C * N * sweeps, res, dict(
        kernel="csr_half_kernel", bytes_per_launch=(2 * C * N + 4 * N + 16 * E) / K,
        traffic="csr_half_kernel_c3_traffic.txt", valu="csr_half_kernel_c3_valu.txt",
        timing_step=lambda i: step(-1 - i), extra=lambda: {},
        energy=lambda: th.ising_energy(prog, st),
        cpu=lambda: cpu_ising(ebm, blocks, args.cpu_seconds, False),
        parity=lambda: parity_spin(th, prog, ebm, blocks, th.hinton_init(th.RngKey(c["key"]), prog, C)
                                   .get_global(), keys[0].seed, 2))


def workload_c4(args, th, wl, torch):
    c = wl.CONFIGS[4]
    C, sweeps, q = c["chains"], c["sweeps"], c["q"]
    n, edges, W, bias, blocks = wl.potts_lattice(c["L"], q, c["w_std"], c["b_std"])
    E = edges.shape[0]
    dev = th.Device(0)
    prog = th.CategoricalProgram(n, q, edges, W, bias, blocks, dev)
    st = prog.new_state(C)
    keys = th.RngKey(c["key"]).split(_n_keys(args))
    step = _run_blocks_workload(th, dev, prog, st, sweeps, keys)
    res = {"config": {"workload": "potts_lattice_512_q8_c32_200sweeps", "L": c["L"], "q": q,
                      "chains": C, "sweeps_per_step": sweeps}, "dtype": "f32"}
    return dev, step, C * n * sweeps, res, dict(
        kernel="potts_pad_kernel",
        bytes_per_launch=(2 * C * n + 4 * q * n + 4 * q * q * E) / 2.0,
        traffic="potts_pad_kernel_c4_traffic.txt",
        valu="potts_pad_kernel_c4_valu.txt", timing_step=lambda i: step(-1 - i), extra=lambda: {},
        energy=lambda: th.potts_energy(prog, st),
        cpu=lambda: cpu_potts(n, q, edges, W, bias, blocks, args.cpu_seconds),
        parity=lambda: parity_potts(th, prog, n, q, edges, W, bias, blocks,
                                    _random_state(C, n, q, 4), keys[0].seed, 2))


def workload_c5(args, th, wl, torch):
    c = wl.CONFIGS[5]
    C, sweeps, V, H = c["chains"], c["sweeps"], c["V"], c["H"]
    bits, Wf, bv, bh = wl.rbm(V, H, c["w_std"], c["b_std"])
    dev = th.Device(0)
    prog = th.RbmProgram(bits, bv, bh, c["beta"], dev)
    st = th.hinton_init(th.RngKey(c["key"]), prog, C)
    keys = th.RngKey(c["key"] + 1).split(_n_keys(args))
    step = _run_blocks_workload(th, dev, prog, st, sweeps, keys)
    res = {"config": {"workload": "rbm_dense_1024x4096_c4096_200sweeps", "visible": V,
                      "hidden": H, "chains": C, "sweeps_per_step": sweeps}, "dtype": "bf16"}
    return dev, step, C * (V + H) * sweeps, res, dict(
        kernel="dense_half_kernel", flops_per_launch=4.0 * C * V * H / 2.0,
        traffic="dense_half_kernel_c5_traffic.txt", mfma_busy="dense_half_kernel_c5_mfma.txt",
        valu="dense_half_kernel_c5_valu.txt", timing_step=lambda i: step(-1 - i),
        extra=lambda: {}, energy=lambda: th.ising_energy(prog, st),
        cpu=lambda: cpu_rbm(Wf, bv, bh, c["beta"], args.cpu_seconds),
        parity=lambda: parity_dense(th, prog, Wf, bv, bh, c["beta"],
                                    th.hinton_init(th.RngKey(c["key"]), prog, C).get_global(),
                                    keys[0].seed, 1))


def workload_c5f32(args, th, wl, torch):
    """Config 5's RBM with f32 weights, the reference's IsingEBM type (as an
    f32 SGD step leaves them): each weight is held exactly as three bf16
    pieces, so each half-sweep's product runs three passes over K.  The
    roofline counts the algorithmic 4CVH flops per sweep, as for config 5."""
    c = wl.CONFIGS[5]
    C, sweeps, V, H = c["chains"], c["sweeps"], c["V"], c["H"]
    W, bv, bh = wl.rbm_f32(V, H, c["w_std"], c["b_std"])
    dev = th.Device(0)
    prog = th.RbmProgram(W, bv, bh, c["beta"], dev)
    assert prog.dense_pieces == 3
    st = th.hinton_init(th.RngKey(c["key"]), prog, C)
    keys = th.RngKey(c["key"] + 1).split(_n_keys(args))
    step = _run_blocks_workload(th, dev, prog, st, sweeps, keys)
    res = {"config": {"workload": "rbm_dense_1024x4096_f32_c4096_200sweeps", "visible": V,
                      "hidden": H, "chains": C, "sweeps_per_step": sweeps,
                      "weight_pieces": prog.dense_pieces}, "dtype": "bf16x3"}
    return dev, step, C * (V + H) * sweeps, res, dict(
        kernel="dense_half_kernel", flops_per_launch=4.0 * C * V * H / 2.0,
        traffic="dense_half_kernel_c5f32_traffic.txt", timing_step=lambda i: step(-1 - i),
        extra=lambda: {}, energy=lambda: th.ising_energy(prog, st),
        cpu=lambda: cpu_rbm(W, bv, bh, c["beta"], args.cpu_seconds),
        parity=lambda: parity_dense(th, prog, W, bv, bh, c["beta"],
                                    th.hinton_init(th.RngKey(c["key"]), prog, C).get_global(),
                                    keys[0].seed, 1))


def gemm_reference(torch, c, reps=50):
    """torch.matmul (hipBLASLt) bf16 GEMMs of the RBM half-sweep shapes: the
    visible update [V x H] x [H x C] and the hidden update [H x V] x [V x C],
    random operands, no sampling."""
    out = {}
    V, H, C = c["V"], c["H"], c["chains"]
    for name, (M, K) in (("visible", (V, H)), ("hidden", (H, V))):
        A = torch.randn(M, K, device="cuda", dtype=torch.bfloat16)
        B = torch.randn(K, C, device="cuda", dtype=torch.bfloat16)
        for _ in range(5):
            A @ B
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            A @ B
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / reps
        tf = 2.0 * M * K * C / dt / 1e12
        out[name] = {"us": dt * 1e6, "TFLOP/s": tf, "frac": tf / BF16_PEAK_TFLOPS}
    return out


def _discrete_bytes(C, n, factors):
    """B_alg per sweep of a discrete factor program: int8 state read and
    written once per chain, every weight and every factor node reference once."""
    w = sum(int(f.weights.size) for f in factors)
    refs = sum(int(f.nodes.size) for f in factors)
    return 2 * C * n + 4 * w + 4 * refs


def workload_d4(args, th, wl, torch):
    """Config 4's Potts model written as CategoricalEBMFactors (bias and pair
    factors) through FactorSamplingProgram: the general discrete kernel on
    the model the role-padded categorical kernel runs (same samples)."""
    import numpy as np

    c = wl.CONFIGS[4]
    C, sweeps, q = c["chains"], c["sweeps"], c["q"]
    n, edges, W, bias, blocks = wl.potts_lattice(c["L"], q, c["w_std"], c["b_std"])
    dev = th.Device(0)
    fs = [th.CategoricalEBMFactor([np.arange(n)], bias.reshape(n, q, 1)),
          th.CategoricalEBMFactor([edges[:, 0], edges[:, 1]], W)]
    prog = th.FactorSamplingProgram(np.ones(n, np.uint8), q, fs, blocks, [], dev)
    st = prog.new_state(C)
    keys = th.RngKey(c["key"]).split(_n_keys(args))
    step = _run_blocks_workload(th, dev, prog, st, sweeps, keys)
    res = {"config": {"workload": "potts_lattice_512_q8_c32_200sweeps_as_factors", "L": c["L"],
                      "q": q, "chains": C, "sweeps_per_step": sweeps, "blocks": 2},
           "dtype": "f32"}
    return dev, step, C * n * sweeps, res, dict(
        kernel="discrete_half_kernel", bytes_per_launch=_discrete_bytes(C, n, fs) / 2.0,
        traffic="discrete_half_kernel_d4_traffic.txt", valu="discrete_half_kernel_d4_valu.txt",
        timing_step=lambda i: step(-1 - i), extra=lambda: {},
        energy=lambda: th.discrete_energy(prog, st),
        cpu=lambda: cpu_discrete(n, np.ones(n, np.uint8), q, fs, [b.nodes for b in blocks],
                                 args.cpu_seconds),
        parity=lambda: parity_discrete(th, prog, n, np.ones(n, np.uint8), q, fs,
                                       [b.nodes for b in blocks], _random_state(C, n, q, 5),
                                       keys[0].seed, 2))


def workload_dmix(args, th, wl, torch):
    """A mixed spin / categorical model (workloads.mixed_lattice(512, 4)) through
    FactorSamplingProgram: spin and categorical blocks of the general
    discrete kernel, square and spin-categorical factors included."""
    C, sweeps, q = 32, 100, 4
    n, kinds, fs, blocks = wl.mixed_lattice(512, q)
    dev = th.Device(0)
    prog = th.FactorSamplingProgram(kinds, q, fs, blocks, [], dev)
    st = prog.new_state(C)
    keys = th.RngKey(5).split(_n_keys(args))
    step = _run_blocks_workload(th, dev, prog, st, sweeps, keys)
    res = {"config": {"workload": "mixed_lattice_512x2_q4_c32_100sweeps", "L": 512, "q": q,
                      "nodes": n, "chains": C, "sweeps_per_step": sweeps, "blocks": 4},
           "dtype": "f32"}
    return dev, step, C * n * sweeps, res, dict(
        kernel="discrete_half_kernel", bytes_per_launch=_discrete_bytes(C, n, fs) / 4.0,
        traffic="discrete_half_kernel_dmix_traffic.txt", valu="discrete_half_kernel_dmix_valu.txt",
        timing_step=lambda i: step(-1 - i), extra=lambda: {},
        energy=lambda: th.discrete_energy(prog, st),
        cpu=lambda: cpu_discrete(n, kinds, q, fs, blocks, args.cpu_seconds),
        parity=lambda: parity_discrete(th, prog, n, kinds, q, fs, blocks,
                                       _random_state(C, n, q, 6, kinds), keys[0].seed, 2))


def workload_w32(args, th, wl, torch):
    """A Potts model with more categories than the narrow kernels take: 256^2
    torus, q = 32 (workloads.potts_lattice), 32 chains, through
    CategoricalProgram on the wide kernel."""
    L, q, C, sweeps = 256, 32, 32, 50
    n, edges, W, bias, blocks = wl.potts_lattice(L, q, 0.2, 0.1)
    E = edges.shape[0]
    dev = th.Device(0)
    prog = th.CategoricalProgram(n, q, edges, W, bias, blocks, dev)
    st = prog.new_state(C)
    keys = th.RngKey(32).split(_n_keys(args))
    step = _run_blocks_workload(th, dev, prog, st, sweeps, keys)
    res = {"config": {"workload": "potts_lattice_256_q32_c32_50sweeps", "L": L, "q": q,
                      "chains": C, "sweeps_per_step": sweeps}, "dtype": "f32"}
    return dev, step, C * n * sweeps, res, dict(
        kernel="potts_wide_kernel",
        bytes_per_launch=(2 * C * n + 4 * q * n + 4 * q * q * E) / 2.0,
        traffic="potts_wide_kernel_w32_traffic.txt", valu="potts_wide_kernel_w32_valu.txt",
        timing_step=lambda i: step(-1 - i), extra=lambda: {},
        energy=lambda: th.potts_energy(prog, st),
        cpu=lambda: cpu_potts(n, q, edges, W, bias, blocks, args.cpu_seconds),
        parity=lambda: parity_potts(th, prog, n, q, edges, W, bias, blocks,
                                    _random_state(C, n, q, 7), keys[0].seed, 2))


WORKLOADS = {"c1": workload_c1, "c2": workload_c2, "c3": workload_c3, "c4": workload_c4,
             "c5": workload_c5}
# programs of the widened rows (general discrete factors; categorical nodes
# with more than 16 categories), reported beside the configurations in the
# default run's `widened` object
WIDENED = {"d4": workload_d4, "dmix": workload_dmix, "w32": workload_w32,
           "c5f32": workload_c5f32}


def _cpu_host():
    """nproc and model name of the host the CPU leg runs on."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "cpu_model": model,
            "omp_num_threads_env": os.environ.get("OMP_NUM_THREADS")}


def cpu_opbyop(ebm, blocks, target_s):
    """The oracle in the reference's op order (materialised [n, k] passes per
    block, crates/thrml-samplers/src/program.rs:324-393), one chain, one
    thread."""
    import numpy as np

    orc = _oracle()
    o = orc.Ising(ebm.n_nodes, ebm.edges, ebm.biases, ebm.weights, ebm.beta,
                  [b.nodes for b in blocks])
    init = np.zeros((1, ebm.n_nodes), np.uint8)
    sweeps, dt = _scaled_sample(lambda k: o.run_blocks_opbyop(7, init, k), target_s, 1)
    return {"value": ebm.n_nodes * sweeps / dt, "unit": "node-updates/s", "cores": 1,
            "kind": "port",
            "sample": f"oracle in the reference's op-by-op order, 1 chain, 1 thread, "
                      f"run_blocks {sweeps} sweeps ({dt:.1f} s)"}


def _parity(name, info):
    """The workload's parity replay (untimed; the CPU side is the oracle)."""
    t0 = time.perf_counter()
    rec = info["parity"]()
    rec["replay_s"] = round(time.perf_counter() - t0, 2)
    ok = rec.get("identical_except_threshold_sites", rec["identical"])
    print(f"bench: {name} parity: {'identical' if rec['identical'] else 'equal except at threshold sites' if ok else 'DIFFERS'}"
          f" ({rec['chains_checked']} chains x {rec['sweeps']} sweeps, "
          f"{rec['threshold_sites']} threshold sites, {rec['replay_s']} s)", file=sys.stderr, flush=True)
    return rec


def measure(name, args, th, wl, torch, steps, warmup, timing=True):
    """Builds workload `name`, runs `warmup` untimed steps and times `steps`
    steps; with timing, also the sweep kernel's average launch (HIP events on
    the library stream) and its rooflines.  Returns (result, device, info)."""
    dev, step, updates_per_step, res, info = {**WORKLOADS, **WIDENED}[name](args, th, wl, torch)
    torch.cuda.synchronize()
    dev.synchronize()
    for i in range(warmup):
        step(i)
    dev.synchronize()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(warmup + i)
    dev.synchronize()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    out = {"value": updates_per_step * steps / dt, "ms_per_step": dt / steps * 1e3,
           "steps": steps, "warmup": warmup, "dtype": res["dtype"], "config": res["config"]}
    if not timing:
        return out, dev, info
    k_ms, k_n = kernel_time(dev, info["timing_step"])
    if "flops_per_launch" in info:
        achieved = info["flops_per_launch"] / (k_ms * 1e-3) / 1e12
        out["roofline"] = {"bound": "mfma", "achieved": achieved, "peak": BF16_PEAK_TFLOPS,
                           "unit": "TFLOP/s", "frac": achieved / BF16_PEAK_TFLOPS,
                           "traffic": _traffic_from_profiles(info["traffic"])
                           if info["traffic"] else None}
        if info.get("mfma_busy"):
            # SQ_VALU_MFMA_BUSY_CYCLES over GRBM_GUI_ACTIVE x SIMDs, committed profile
            out["roofline"]["mfma_busy_counter"] = _profile_value(info["mfma_busy"],
                                                                  "mfma_busy_frac")
    else:
        achieved = info["bytes_per_launch"] / (k_ms * 1e-3) / 1e9
        out["roofline"] = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS,
                           "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
                           "traffic": _traffic_from_profiles(info["traffic"])
                           if info["traffic"] else None}
    # the sweep kernels are VALU-bound (keystream, decisions): the same launch
    # against the vector-ALU issue peak, from the committed instruction counts
    valu = _profile_value(info["valu"], "valu_instr_per_launch") if info.get("valu") else None
    if valu:
        g = valu / (k_ms * 1e-3) / 1e9
        out["valu_roofline"] = {"achieved": g, "peak": VALU_PEAK_GWIS,
                                "unit": "G wave-instructions/s", "frac": g / VALU_PEAK_GWIS,
                                "instr_per_launch": valu}
    out["kernel_us"] = {info["kernel"]: k_ms * 1e3, "launches": k_n}
    return out, dev, info


# steps per configuration in the `configs` object of the default run (each
# step is the configuration's full sweep count; about 1-2 s of GPU time each)
CONFIG_STEPS = {"c1": 20, "c2": 5, "c3": 5, "c4": 10, "c5": 10, "d4": 3, "dmix": 3, "w32": 5,
                "c5f32": 3}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", choices=sorted(WORKLOADS) + sorted(WIDENED), default="c2")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="first run a plain device-to-device copy of this many MiB (the "
                         "known-size reference for rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the event-timed pass and the extra passes")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other configurations' measurements")
    ap.add_argument("--energy", type=int, default=0, metavar="N",
                    help="also time N per-chain energy evaluations of the final state")
    ap.add_argument("--gemm-reference", action="store_true",
                    help="c5: also time torch.matmul (hipBLASLt) bf16 GEMMs of the two "
                         "half-sweep shapes")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU.  The sweep shards over chains with no "
              "communication until a final moment all-reduce, which is not built here.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import thrml_hip as th
    from thrml_hip import workloads as wl

    if args.copy_mib:
        a = torch.ones(args.copy_mib << 18, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        b.copy_(a)
        torch.cuda.synchronize()
        del a, b

    head, dev, info = measure(args.workload, args, th, wl, torch, args.steps, args.warmup,
                              timing=not args.no_extra)
    result = {
        "metric": "node-updates/s",
        "value": head["value"],
        "unit": "node-updates/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": head["dtype"],
        "data": "synthetic",
        "config": head["config"],
    }
    if args.energy:
        info["energy"]()  # first call: builds the energy tables
        dev.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.energy):
            info["energy"]()
        result["energy_ms_per_call"] = (time.perf_counter() - t0) / args.energy * 1e3
    if args.gemm_reference and args.workload == "c5":
        result["gemm_reference"] = gemm_reference(torch, wl.CONFIGS[5])
    if args.no_extra:
        print(json.dumps(result))
        return
    for k in ("roofline", "valu_roofline", "kernel_us"):
        if k in head:
            result[k] = head[k]
    result.update(info["extra"]())
    cpu = None if args.no_cpu else info["cpu"]()
    if cpu is not None:
        cpu.update(_cpu_host())
        if "opbyop" in info:
            cpu["op_by_op_1_thread"] = info["opbyop"]()
        result["cpu_baseline"] = cpu
        result["parity"] = _parity(args.workload, info)
    if not args.no_configs:
        # every other configuration, measured the same way in this run
        configs = {}
        dev.close()
        for name in sorted(WORKLOADS):
            if name == args.workload:
                continue
            r, d, inf = measure(name, args, th, wl, torch, CONFIG_STEPS[name], 1)
            configs[name] = {k: r[k] for k in ("value", "ms_per_step", "steps", "warmup",
                                               "dtype", "roofline", "valu_roofline",
                                               "kernel_us") if k in r}
            configs[name]["workload"] = r["config"]["workload"]
            if not args.no_cpu:
                configs[name]["parity"] = _parity(name, inf)
            d.close()
            print(f"bench: {name} {r['value']:.4g} node-updates/s, "
                  f"{r['roofline']['bound']} frac {r['roofline']['frac']:.3f}",
                  file=sys.stderr, flush=True)
        result["configs"] = configs
        widened = {}
        for name in sorted(WIDENED):
            if name == args.workload:
                continue
            r, d, inf = measure(name, args, th, wl, torch, CONFIG_STEPS[name], 1)
            widened[name] = {k: r[k] for k in ("value", "ms_per_step", "steps", "warmup",
                                               "dtype", "roofline", "valu_roofline",
                                               "kernel_us") if k in r}
            widened[name]["workload"] = r["config"]["workload"]
            if not args.no_cpu:
                widened[name]["parity"] = _parity(name, inf)
            d.close()
            print(f"bench: {name} {r['value']:.4g} node-updates/s, "
                  f"{r['roofline']['bound']} frac {r['roofline']['frac']:.3f}",
                  file=sys.stderr, flush=True)
        result["widened"] = widened
    print(json.dumps(result))


if __name__ == "__main__":
    main()
