"""Pins of the oracle's dense bipartite (RBM) half-sweep (oracle/orc_rbm.c).

An RBM is an IsingEBM on the complete bipartite graph with edges (v, V + h)
in the order e = v*H + h (crates/thrml-models/src/ising.rs:26-143); the
Ising oracle is pinned independently (energy identity, exact enumeration).
The RBM oracle sums the products in double and rounds once, so its
decisions must equal `u <= sigmoid(2 * gamma)` with gamma from the Ising
oracle's slot-order f32 sum everywhere except at its flagged threshold
sites.  A transposed weight matrix or a flipped sign is planted to show that
the comparison has the power to catch those mistakes."""
import numpy as np
import pytest

import pyoracle as orc


def _model(V, H, seed):
    rng = np.random.default_rng(seed)
    W = rng.normal(0, 0.5, (V, H)).astype(np.float32)
    bv = rng.normal(0, 0.3, V).astype(np.float32)
    bh = rng.normal(0, 0.3, H).astype(np.float32)
    return rng, W, bv, bh


def _ising_decisions(W, bv, bh, beta, key8, blk, sv, sh):
    V, H = W.shape
    edges = np.array([(v, V + h) for v in range(V) for h in range(H)], np.uint32)
    ising = orc.Ising(V + H, edges, np.concatenate([bv, bh]), W.reshape(-1), beta,
                      [np.arange(V), np.arange(V, V + H)])
    n, off = (V, 0) if blk == 0 else (H, V)
    out = np.zeros((sv.shape[0], n), np.uint8)
    for c in range(sv.shape[0]):
        g = ising.gamma(np.concatenate([sv[c], sh[c]]))[off:off + n]
        u = np.array([(orc.stream_word(key8[c], i) >> 8) * 2.0**-24 for i in range(n)], np.float32)
        p = orc.map_f32("sigmoid", (2.0 * g).astype(np.float32))
        out[c] = u <= p
    return out


@pytest.mark.parametrize("V,H,blk", [(12, 20, 0), (12, 20, 1), (7, 33, 0), (33, 7, 1)])
def test_rbm_oracle_matches_ising_oracle(V, H, blk):
    rng, W, bv, bh = _model(V, H, V * 100 + H + blk)
    C, beta = 6, 0.8
    sv = rng.integers(0, 2, (C, V)).astype(np.uint8)
    sh = rng.integers(0, 2, (C, H)).astype(np.uint8)
    key8 = rng.integers(0, 2**32, (C, 8), dtype=np.uint64).astype(np.uint32)
    ov, oh, near = orc.rbm_half_sweep(W, bv, bh, beta, key8, blk, sv, sh)
    got = ov if blk == 0 else oh
    want = _ising_decisions(W, bv, bh, beta, key8, blk, sv, sh)
    assert np.array_equal(got[near == 0], want[near == 0])
    # the other block is untouched
    assert np.array_equal(oh if blk == 0 else ov, sh if blk == 0 else sv)


@pytest.mark.parametrize("mistake", ["transpose", "sign", "wrong_bias"])
def test_planted_mistakes_are_detected(mistake):
    V, H, blk = 16, 16, 0
    rng, W, bv, bh = _model(V, H, 5)
    W *= 3.0  # strong couplings: decisions follow gamma closely
    C, beta = 8, 1.0
    sv = rng.integers(0, 2, (C, V)).astype(np.uint8)
    sh = rng.integers(0, 2, (C, H)).astype(np.uint8)
    key8 = rng.integers(0, 2**32, (C, 8), dtype=np.uint64).astype(np.uint32)
    if mistake == "transpose":
        ov, _, _ = orc.rbm_half_sweep(np.ascontiguousarray(W.T), bv, bh, beta, key8, blk, sv, sh)
    elif mistake == "sign":
        ov, _, _ = orc.rbm_half_sweep(W, bv, bh, beta, key8, blk, sv, 1 - sh)
    else:
        ov, _, _ = orc.rbm_half_sweep(W, bv * 0 + 4.0, bh, beta, key8, blk, sv, sh)
    want = _ising_decisions(W, bv, bh, beta, key8, blk, sv, sh)
    assert (ov != want).sum() >= 10
