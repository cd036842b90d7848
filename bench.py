"""Benchmark of the block Gibbs sweep on one MI355X.

Workload: 1024 x 1024 periodic Ising lattice,
checkerboard 2-block Gibbs, biases ~N(0, 0.1), couplings ~N(0.44, 0.05),
beta = 1, 64 chains, 500 sweeps with magnetisation and nearest-neighbour
moments observed (schedule n_warmup=1, n_samples=500, steps_per_sample=1).
One step = one sample_with_observation run of that schedule through a
MomentAccumulatorObserver built once for all nodes and all edges, with the
chains resident in HBM before the timed region starts and the exact moment
sums left in device memory (as the reference leaves its moments in device
tensors).

metric: node-updates/s = chains * nodes * sweeps / time.
roofline: the lattice half-sweep kernel; algorithmic bytes per launch =
  (2*C*N + 4*N + 4*E) / 2 (int8-equivalent state read + written once per
  chain, parameters once, indices implicit, per half-sweep), divided by the
  kernel's average duration from HIP events recorded on the library stream.
  traffic: HBM bytes per launch from the committed rocprofv3 counter summary.
cpu_baseline: the CPU oracle (a C restatement of the reference's sweep and
  moment observer), OpenMP over chains, on a bounded sample of the same
  program: fewer chains and sweeps, same 1024^2 lattice and schedule shape.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "thrml-rs_amd"))

HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "lattice_half_kernel_c2_traffic.txt")


def _traffic_from_profiles():
    """HBM bytes per launch of the half-sweep kernel (FETCH_SIZE + WRITE_SIZE,
    calibrated) from the committed rocprofv3 summary, if present."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    with open(TRAFFIC_FILE) as f:
        for line in f:
            if line.startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1])
    return None


def cpu_baseline(ebm, blocks, target_s=15.0):
    """Oracle sample_with_observation + moments on host cores over a bounded
    sample; returns node-updates/s."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import numpy as np

    import pyoracle as orc

    o = orc.Ising(ebm.n_nodes, ebm.edges, ebm.biases, ebm.weights, ebm.beta,
                  [b.nodes for b in blocks])
    threads = orc.threads()
    n = ebm.n_nodes
    nodes = np.arange(n, dtype=np.uint32)
    init = np.zeros((threads, n), np.uint8)
    t0 = time.perf_counter()
    o.estimate_moments(7, (1, 2, 1), init, nodes, ebm.edges, threads)
    dt2 = time.perf_counter() - t0
    sweeps = max(2, int(target_s / max(dt2 / 2, 1e-3)))
    t0 = time.perf_counter()
    o.estimate_moments(7, (1, sweeps, 1), init, nodes, ebm.edges, threads)
    dt = time.perf_counter() - t0
    rate = threads * n * sweeps / dt
    return {"value": rate, "unit": "node-updates/s", "cores": threads, "kind": "port",
            "sample": f"oracle estimate_moments on the 1024^2 config-2 program: {threads} chains "
                      f"(one per thread) x {sweeps} sweeps, schedule (1, {sweeps}, 1), all node "
                      f"and edge moments ({dt:.1f} s)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="first run a plain device-to-device copy of this many MiB (the "
                         "known-size reference for rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the event-timed pass and the sweep-only pass")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py: this build runs on one GPU.  The sweep shards over chains with no "
              "communication until a final moment all-reduce, which is not built here.",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import thrml_hip as th
    from thrml_hip import workloads as wl

    if args.copy_mib:
        a = torch.ones(args.copy_mib << 18, dtype=torch.float32, device="cuda")
        b = torch.empty_like(a)
        b.copy_(a)
        torch.cuda.synchronize()
        del a, b

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
    run_keys = k_run.split(args.warmup + args.steps + 2)
    torch.cuda.synchronize()
    dev.synchronize()

    def step(k):
        observer.sample_with_observation(k, sched, st, out=out)

    for i in range(args.warmup):
        step(run_keys[i])
    dev.synchronize()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(run_keys[args.warmup + i])
    dev.synchronize()
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ms_per_step = dt / args.steps * 1e3
    value = C * N * sweeps * args.steps / dt

    if args.no_extra:
        print(json.dumps({"metric": "node-updates/s", "value": value, "ms_per_step": ms_per_step}))
        return

    # per-launch durations from HIP events on the library stream
    dev.enable_timing(True)
    for k in run_keys[-2:]:
        step(k)
    dev.synchronize()
    k_ms, k_n = dev.kernel_time(0)
    m_ms, m_n = dev.kernel_time(1)
    dev.enable_timing(False)
    b_alg_launch = (2 * C * N + 4 * N + 4 * E) / 2.0
    achieved = b_alg_launch / (k_ms * 1e-3) / 1e9

    # the sweep alone (run_blocks, no observation), same chains and sweeps
    t0 = time.perf_counter()
    th.run_blocks(th.RngKey(99), prog, st, (), sweeps)
    dev.synchronize()
    sweep_only = C * N * sweeps / (time.perf_counter() - t0)

    result = {
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
        "kernel_us": {"lattice_half_kernel": k_ms * 1e3, "launches": k_n,
                      "moment_kernels": m_ms * 1e3, "moment_launches": m_n},
        "sweep_only_node_updates_per_s": sweep_only,
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(ebm, blocks, args.cpu_seconds)
    print(json.dumps(result))


if __name__ == "__main__":
    main()
