"""Benchmark of the block Gibbs sweep on one MI355X.

Workload: 1024 x 1024 periodic Ising lattice,
checkerboard 2-block Gibbs, biases ~N(0, 0.1), couplings ~N(0.44, 0.05),
beta = 1, 64 chains, 500 sweeps with magnetisation and nearest-neighbour
moments observed (schedule n_warmup=1, n_samples=500, steps_per_sample=1).
One step = one estimate_moments call over that schedule, with the chains
resident in HBM before the timed region starts.

metric: node-updates/s = chains * nodes * sweeps / time.
roofline: the lattice half-sweep kernel; algorithmic bytes per launch =
  (2*C*N + 4*N + 4*E) / 2 (int8 state read + written once per chain,
  parameters once, per half-sweep), divided by the kernel's average duration
  from HIP events on the library stream.
cpu_baseline: the CPU oracle (a port of the reference's sweep), timed on a
  bounded sample of the same workload on this host.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "thrml-rs_amd"))

HBM_PEAK_GBS = 8000.0


def _traffic_from_profiles():
    """HBM bytes per launch of the half-sweep kernel from the committed
    rocprofv3 counter summary (profiles/), if present."""
    path = os.path.join(ROOT, "profiles", "lattice_half_kernel_c2_counters.json")
    if not os.path.exists(path):
        return None
    try:
        with open(path) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    except Exception:
        return None


def cpu_baseline(ebm, blocks, C, target_s=12.0):
    """Oracle run_blocks on host cores over a bounded sample (a few chains of
    the same 1024^2 program); returns node-updates/s."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np

    import pyoracle as orc

    o = orc.Ising(ebm.n_nodes, ebm.edges, ebm.biases, ebm.weights, ebm.beta,
                  [b.nodes for b in blocks])
    threads = orc.threads()
    n = ebm.n_nodes
    init = np.zeros((threads, n), np.uint8)
    t0 = time.perf_counter()
    o.run_blocks_subset(42, C, list(range(threads)), init, 1, threads)
    dt1 = time.perf_counter() - t0
    sweeps = max(1, int(target_s / max(dt1, 1e-3)))
    t0 = time.perf_counter()
    o.run_blocks_subset(42, C, list(range(threads)), init, sweeps, threads)
    dt = time.perf_counter() - t0
    rate = threads * n * sweeps / dt
    return {"value": rate, "unit": "node-updates/s", "cores": threads, "kind": "port",
            "sample": f"oracle run_blocks, {threads} chains x {n} nodes x {sweeps} sweeps of the "
                      f"1024^2 config-2 program ({dt:.1f} s, one chain per thread)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU only (chains shard across GPUs with no "
              "communication until a final moment all-reduce; not built here).", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import thrml_hip as th
    from thrml_hip import workloads as wl

    c = wl.CONFIGS[2]
    C, sweeps = c["chains"], c["sweeps"]
    ebm, blocks = wl.config_ising(2)
    N, E = ebm.n_nodes, ebm.edge_u.size
    dev = th.Device(0)
    prog = th.IsingSamplingProgram(ebm, blocks, [], dev)
    assert prog.kind == "lattice"
    sched = th.SamplingSchedule(1, sweeps, 1)
    nodes = np.arange(N, dtype=np.uint32)
    edges = ebm.edges
    k_init, k_run = th.RngKey(c["key"]).split_two()
    st = th.hinton_init(k_init, prog, C)
    dev.synchronize()

    def step(i):
        th.estimate_moments(th.RngKey(k_run.seed + i), nodes, edges, prog, sched, st,
                            return_sums=True)

    for i in range(args.warmup):
        step(i)
    dev.synchronize()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(args.warmup + i)
    dev.synchronize()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms_per_step = dt / args.steps * 1e3
    updates = C * N * sweeps * args.steps
    value = updates / dt

    # second timed pass with per-launch HIP events on the library stream
    dev.enable_timing(True)
    for i in range(max(1, args.steps // 2)):
        step(1000 + i)
    dev.synchronize()
    k_ms, k_n = dev.kernel_time(0)
    m_ms, m_n = dev.kernel_time(1)
    dev.enable_timing(False)
    b_alg_launch = (2 * C * N + 4 * N + 4 * E) / 2.0
    achieved = b_alg_launch / (k_ms * 1e-3) / 1e9

    out = {
        "metric": "node-updates/s",
        "value": value,
        "unit": "node-updates/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "ising_lattice_1024_c64_500sweeps_moments", "L": 1024,
                   "chains": C, "sweeps_per_step": sweeps, "blocks": 2,
                   "schedule": [1, sweeps, 1], "moments": "all nodes + all edges"},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": _traffic_from_profiles()},
        "kernel_ms": {"lattice_half_kernel": k_ms, "launches": k_n,
                      "moments_kernel": m_ms, "moment_launches": m_n},
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(ebm, blocks, C)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
