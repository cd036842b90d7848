"""Configurations 2, 3 and 4 run for their full configured length on the
device, bit for bit against the oracle: the oracle's initial state, final
state and (config 2) int64 moment sums are kept as SHA-256 digests in
tests/golden/full_runs.json, which tests/golden/make_full_runs.py writes (the
oracle needs minutes for these runs, the device milliseconds).

  - config 2: the bench's observer path, hinton_init then every node and
    edge moment over schedule (1, 500, 1) (ising.rs:455-505, 602-673);
  - config 3: the 1M-node Erdos-Renyi program, hinton_init then 200 sweeps of
    run_blocks over its 10 colour blocks (sampling.rs:81-126);
  - config 4: the q = 8 Potts torus from a seeded random state, 200 sweeps.
Every chain and every site of the final state is covered by its digest."""
import hashlib
import json
import os

import numpy as np
import pytest

import thrml_hip as th
from conftest import log_case
from thrml_hip import workloads as wl

pytestmark = pytest.mark.gpu

GOLDEN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "full_runs.json")))


def _digest(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_config2_full_run_moments_and_state(device):
    import torch

    g = GOLDEN["c2"]
    ebm, blocks = wl.config_ising(2)
    N = ebm.n_nodes
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    assert prog.kind == "lattice"
    k_init, k_run = th.RngKey(wl.CONFIGS[2]["key"]).split_two()
    assert (k_init.seed, k_run.seed) == (g["init_key"], g["run_key"])
    log_case(f"config2 full run: schedule {g['schedule']}, {g['chains']} chains")
    st = th.hinton_init(k_init, prog, g["chains"])
    assert _digest(st.get_global()) == g["init"]
    observer = th.MomentAccumulatorObserver(
        prog, th.ising_moment_spec(np.arange(N, dtype=np.uint32), ebm.edges))
    out = (torch.empty(N, dtype=torch.int64, device="cuda"),
           torch.empty(ebm.edges.shape[0], dtype=torch.int64, device="cuda"))
    torch.cuda.synchronize()
    observer.sample_with_observation(k_run, th.SamplingSchedule(*g["schedule"]), st, out=out)
    device.synchronize()
    assert _digest(st.get_global()) == g["final"]
    assert _digest(out[0].cpu().numpy().astype(np.int64)) == g["node_sums"]
    assert _digest(out[1].cpu().numpy().astype(np.int64)) == g["edge_sums"]
    observer.close()
    st.close()


def test_config3_full_run(device):
    g = GOLDEN["c3"]
    ebm, blocks = wl.config3()
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    assert prog.kind == "csr"
    log_case(f"config3 full run: {g['sweeps']} sweeps, {g['chains']} chains, {len(blocks)} blocks")
    st = th.hinton_init(th.RngKey(g["init_key"]), prog, g["chains"])
    assert _digest(st.get_global()) == g["init"]
    th.run_blocks(th.RngKey(g["run_key"]), prog, st, (), g["sweeps"])
    assert _digest(st.get_global()) == g["final"]
    st.close()


def test_config4_full_run(device):
    g = GOLDEN["c4"]
    c = wl.CONFIGS[4]
    n, edges, W, bias, blocks = wl.potts_lattice(c["L"], c["q"], c["w_std"], c["b_std"])
    prog = th.CategoricalProgram(n, c["q"], edges, W, bias, blocks, device)
    log_case(f"config4 full run: {g['sweeps']} sweeps, {g['chains']} chains")
    init = np.random.default_rng(g["init_seed"]).integers(0, c["q"], (g["chains"], n)).astype(np.uint8)
    assert _digest(init) == g["init"]
    st = prog.new_state(g["chains"])
    st.set_global(init)
    th.run_blocks(th.RngKey(g["run_key"]), prog, st, (), g["sweeps"])
    assert _digest(st.get_global()) == g["final"]
    st.close()
