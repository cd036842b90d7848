"""10,000-sweep moment runs against the oracle (north_star: per-node
magnetisation and pairwise moments agree within 1e-3 over 10k sweeps, with
sites whose pre-activation lies within 1e-5 of the threshold counted and
reported).

The GPU and the oracle draw the same keyed uniforms and evaluate the same
decision math, so the trajectories are identical and the integer moment sums
agree exactly; the 1e-3 bound on the means is asserted as well, and the
oracle's threshold-site count (against its libm-free sigmoid, so expected 0)
is printed.  Cases: config 1's model (64 x 64 torus, b ~ N(0, 0.1),
J ~ N(0.3, 0.05), hinton init, RngKey(42)) and an Erdos-Renyi graph of 2000
nodes with mean degree 12 and greedy-colour blocks (the CSR kernel), 32
chains each, schedule (1, 10000, 1), every node and every edge observed."""
import numpy as np
import pytest

import pyoracle as orc
import thrml_hip as th
from conftest import log_case
from thrml_hip import workloads as wl

pytestmark = pytest.mark.gpu

C = 32
SCHED = (1, 10000, 1)


def _run(device, ebm, blocks):
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    o = orc.Ising(ebm.n_nodes, ebm.edges, ebm.biases, ebm.weights, ebm.beta,
                  [b.nodes for b in blocks])
    k_init, k_run = th.RngKey(42).split_two()
    st = th.hinton_init(k_init, prog, C)
    init = st.get_global()
    assert np.array_equal(init, o.hinton_init(k_init.seed, C))
    nodes = np.arange(ebm.n_nodes, dtype=np.uint32)
    ns, es = th.estimate_moments(k_run, nodes, ebm.edges, prog, th.SamplingSchedule(*SCHED), st,
                                 return_sums=True)
    ons, oes, ofinal, thr = o.estimate_moments(k_run.seed, SCHED, init, nodes, ebm.edges)
    n_obs = C * SCHED[1]
    # first moments <s_i> and second moments <s_i s_j> from the +-1 sums
    dm = np.abs(ns.astype(np.float64) - ons.astype(np.float64)).max() / n_obs
    de = np.abs(es.astype(np.float64) - oes.astype(np.float64)).max() / n_obs
    print(f"{prog.kind}: max |d<s_i>| = {dm:.2e}, max |d<s_i s_j>| = {de:.2e}, "
          f"threshold sites counted by the oracle: {thr}")
    assert dm <= 1e-3 and de <= 1e-3
    assert np.array_equal(ns, ons) and np.array_equal(es, oes)
    assert np.array_equal(st.get_global(), ofinal)
    return prog


def test_config1_model_10k_sweeps(device):
    log_case("10k sweeps, config 1 model, 32 chains")
    ebm, blocks = wl.config_ising(1)
    assert _run(device, ebm, blocks).kind == "lattice"


def test_erdos_renyi_10k_sweeps(device):
    log_case("10k sweeps, Erdos-Renyi 2000 nodes, 32 chains")
    ebm, blocks = wl.er_ising(2000, 12.0, 0.2, 0.0, 0.3)
    assert _run(device, ebm, blocks).kind == "csr"


def test_dense_rbm_10k_sweeps_against_exact_moments(device):
    """The dense path sums on the matrix cores, so its decisions may differ from
    the slot-order sum at threshold sites and its trajectories are not the
    oracle's; its moments are checked against exact enumeration instead:
    6 visible + 5 hidden spins (2^11 states), 4096 chains, 10,000 observed
    sweeps, every node and every edge within 1e-3 of the exact Boltzmann
    moments (about 4.5 standard errors at 4.1e7 samples)."""
    from test_gpu_dense import _exact_ising_moments

    log_case("10k sweeps, dense 6 x 5, 4096 chains")
    V, H, Cd = 6, 5, 4096
    rng = np.random.default_rng(21)
    bits, Wf = th.bf16_round(rng.normal(0, 0.3, (V, H)).astype(np.float32))
    bv = rng.normal(0, 0.3, V).astype(np.float32)
    bh = rng.normal(0, 0.3, H).astype(np.float32)
    beta = 1.0
    prog = th.RbmProgram(bits, bv, bh, beta, device)
    edges = np.array([(v, V + h) for v in range(V) for h in range(H)], np.uint32)
    m1, m2 = _exact_ising_moments(V + H, edges, np.concatenate([bv, bh]).astype(np.float64),
                                  Wf.reshape(-1).astype(np.float64), beta)
    st = th.hinton_init(th.RngKey(3), prog, Cd)
    nm, em = th.estimate_moments(th.RngKey(4), np.arange(V + H), edges, prog,
                                 th.SamplingSchedule(20, 10000, 1), st)
    print(f"dense: max |<s_i> - exact| = {np.abs(nm - m1).max():.2e}, "
          f"max |<s_i s_j> - exact| = {np.abs(em - m2).max():.2e}")
    assert np.abs(nm - m1).max() < 1e-3 and np.abs(em - m2).max() < 1e-3
