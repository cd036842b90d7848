"""Writes full_runs.json: digests of the oracle's results for configurations
2, 3 and 4 run for their full configured length, which the GPU tests in
test_gpu_full_runs.py compare against (the oracle takes minutes on these
sizes; the device takes milliseconds).

  - config 2 (1024^2 torus Ising, 64 chains): the bench's observer path,
    hinton_init(split_two(RngKey(42))[0]) then estimate_moments over every
    node and edge with schedule (1, 500, 1) keyed by split_two(RngKey(42))[1]
    (crates/thrml-models/src/ising.rs:455-505, 602-673);
  - config 3 (1M-node Erdos-Renyi Ising, 10 colour blocks, 32 chains):
    hinton_init(RngKey(42)), then run_blocks(RngKey(43), 200 sweeps)
    (crates/thrml-samplers/src/sampling.rs:81-126);
  - config 4 (512^2 torus Potts, q = 8, 32 chains): a seeded random state,
    then run_blocks(RngKey(44), 200 sweeps).

Each entry holds the SHA-256 of the initial state, of the final state (uint8
[chains][n] in global order) and, for config 2, of the int64 moment sums, plus
the count of threshold sites the oracle met (site updates whose decision lies
within 1e-5 of the sampling threshold; the device decides them exactly as the
oracle does).  Run from the repository root with the oracle and the library's
host code built: python tests/golden/make_full_runs.py"""
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [os.path.join(ROOT, "oracle"), os.path.join(ROOT, "thrml-rs_amd")]

import pyoracle as orc  # noqa: E402
from thrml_hip import workloads as wl  # noqa: E402


def digest(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def config2():
    c = wl.CONFIGS[2]
    ebm, blocks = wl.config_ising(2)
    N = ebm.n_nodes
    k_init, k_run = (int(k) for k in orc.rng_split(c["key"], 2))
    o = orc.Ising(N, ebm.edges, ebm.biases, ebm.weights, ebm.beta, [b.nodes for b in blocks])
    init = o.hinton_init(k_init, c["chains"])
    sched = (1, c["sweeps"], 1)
    ns, es, final, near = o.estimate_moments(k_run, sched, init, np.arange(N, dtype=np.uint32),
                                             ebm.edges)
    return {"init_key": k_init, "run_key": k_run, "schedule": list(sched),
            "chains": c["chains"], "init": digest(init), "final": digest(final),
            "node_sums": digest(ns.astype(np.int64)), "edge_sums": digest(es.astype(np.int64)),
            "threshold_sites": int(near), "mean_spin": float(final.mean())}


def config3():
    c = wl.CONFIGS[3]
    ebm, blocks = wl.config3()
    o = orc.Ising(ebm.n_nodes, ebm.edges, ebm.biases, ebm.weights, ebm.beta,
                  [b.nodes for b in blocks])
    init = o.hinton_init(c["key"], c["chains"])
    final, near = o.run_blocks(c["key"] + 1, init, c["sweeps"])
    return {"init_key": c["key"], "run_key": c["key"] + 1, "sweeps": c["sweeps"],
            "chains": c["chains"], "init": digest(init), "final": digest(final),
            "threshold_sites": int(near), "mean_spin": float(final.mean())}


def config4():
    c = wl.CONFIGS[4]
    n, edges, W, bias, blocks = wl.potts_lattice(c["L"], c["q"], c["w_std"], c["b_std"])
    o = orc.Potts(n, c["q"], edges, W, bias, [b.nodes for b in blocks])
    init = np.random.default_rng(4).integers(0, c["q"], (c["chains"], n)).astype(np.uint8)
    final, near = o.run_blocks(c["key"] + 2, init, c["sweeps"])
    return {"init_seed": 4, "run_key": c["key"] + 2, "sweeps": c["sweeps"],
            "chains": c["chains"], "init": digest(init), "final": digest(final),
            "threshold_sites": int(near), "mean_category": float(final.mean())}


def main():
    out = {}
    for name, fn in (("c2", config2), ("c3", config3), ("c4", config4)):
        t0 = time.perf_counter()
        out[name] = fn()
        print(f"{name}: {time.perf_counter() - t0:.1f} s, {out[name]}", flush=True)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "full_runs.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
