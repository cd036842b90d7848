"""The MNIST training set-up of crates/thrml-models/tests/test_train_mnist.rs
on the GPU: the double grid (40 x 40 layers, jumps 1, 4, 15, 814 visible
nodes), zero-initialised IsingEBM, positive phase over (upper without
visible, lower) with the visible block clamped to a data row, negative phase
over (upper, lower), schedules (50, 10, 3), one chain, batches of 10 rows,
keys = key.split(3) per batch, SGD w += 0.01 grad (:386-520).

The reference's training file (train_data_filtered.npy) is not in its
checkout; the rows here are its held test images of the digits 0, 3, 4
(tests/golden/mnist_034_subset.npz) followed by 30 label bits, ten per class
(class k sets bits 784 + 10k .. 784 + 10k + 9).  Every batch's gradients
equal the oracle's, bit for bit, through three SGD steps."""
import os

import numpy as np
import pytest

import pyoracle as orc
import thrml_hip as th
from conftest import log_case

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def mnist_rows():
    z = np.load(os.path.join(HERE, "golden", "mnist_034_subset.npz"), allow_pickle=False)
    imgs = [np.unpackbits(z[f"digit{d}"], axis=1)[:, :784] for d in (0, 3, 4)]
    n = min(len(a) for a in imgs)
    rows = []
    for i in range(n):  # interleave the classes
        for k, a in enumerate(imgs):
            lab = np.zeros(30, np.uint8)
            lab[10 * k:10 * k + 10] = 1
            rows.append(np.concatenate([a[i], lab]))
    return np.array(rows, np.float32)


def test_mnist_double_grid_training_matches_oracle(device):
    side, jumps, data_dim = 40, [1, 4, 15], 28 * 28 + 30
    up, lo, vis, rest, n, edges = th.double_grid(side, jumps, data_dim, 0)
    data = mnist_rows()
    assert data.shape[1] == data_dim
    b = np.zeros(n, np.float32)
    w = np.zeros(edges.shape[0], np.float32)
    pos_blocks, neg_blocks = [rest, lo], [up, lo]
    sched = th.SamplingSchedule(50, 10, 3)
    nodes = np.arange(n, dtype=np.uint32)
    key = th.RngKey(0)
    lr = np.float32(0.01)
    for batch in range(3):
        log_case(f"mnist double grid batch {batch}")
        rows = data[batch * 10:(batch + 1) * 10]
        keys = key.split(3)
        key = keys[2]
        ebm = th.IsingEBM(n, edges, b, w, 1.0)
        spec = th.IsingTrainingSpec(ebm, [vis], [], pos_blocks, neg_blocks, sched, sched, device)
        init_pos = th.hinton_init(keys[0], spec.program_positive, 1)
        init_neg = th.hinton_init(keys[1], spec.program_negative, 1)
        gw, gb = th.estimate_kl_grad(keys[0], spec, nodes, edges, [rows], [], init_pos, init_neg)

        # oracle: the same two phases from the same hinton states and keys
        kp, kn = keys[0].split_two()
        o_pos = orc.Ising(n, edges, b, w, 1.0, [rest.nodes, lo.nodes], [vis.nodes])
        st_pos = o_pos.hinton_init(keys[0].seed, 1)
        nf = len(rest) + len(lo)
        st_pos[:, nf:] = rows[kp.seed % rows.shape[0]].astype(np.uint8)  # visible-block order
        ns_p, es_p, _, _ = o_pos.estimate_moments(kp.seed, (50, 10, 3), st_pos, nodes, edges)
        o_neg = orc.Ising(n, edges, b, w, 1.0, [up.nodes, lo.nodes], [])
        st_neg = o_neg.hinton_init(keys[1].seed, 1)
        ns_n, es_n, _, _ = o_neg.estimate_moments(kn.seed, (50, 10, 3), st_neg, nodes, edges)
        d = np.float32(10)
        want_b = (ns_p.astype(np.float32) / d - ns_n.astype(np.float32) / d) * np.float32(-1.0)
        want_w = (es_p.astype(np.float32) / d - es_n.astype(np.float32) / d) * np.float32(-1.0)
        assert np.array_equal(gb, want_b), batch
        assert np.array_equal(gw, want_w), batch
        assert np.abs(gw).max() > 0
        print(f"batch {batch}: |grad_w| {np.sqrt((gw.astype(np.float64) ** 2).sum()):.3f}, "
              f"|grad_b| {np.sqrt((gb.astype(np.float64) ** 2).sum()):.3f}")
        w = (w + gw * lr).astype(np.float32)
        b = (b + gb * lr).astype(np.float32)
        spec.close()
