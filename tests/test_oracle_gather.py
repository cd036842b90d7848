"""The oracle's batch_gather_fused (crates/thrml-kernels/src/batch_gather/
kernel.rs, launched by batch_gather/forward.rs; the export R14 lists beside
sigmoid-Bernoulli and Gumbel-argmax), pinned without retyping its loop:

  - with C-ordered strides of a weight array of shape [batch, d1, ..., dk]
    and in-range indices, the result is numpy's own multi-dimensional
    indexing weights[b, i1, ..., ik], for k = 1 .. 8 (the reference's tests
    use 2 to 8 indices: mod.rs:26-60, test_batch_gather_extended.rs);
  - the reference's 3-index case (test_batch_gather_extended.rs:12-35) on
    arange weights: element 0 reads entry 22, element 1's linear index 123
    lies past the 120 entries (the reference only checks the length; this
    build reads 0.0 there);
  - the u32 wrapping of the reference's index arithmetic (u32::cast_from of a
    negative index, products and sums modulo 2^32), on arange weights whose
    value is the linear index, against Python integers."""
import numpy as np
import pytest

import pyoracle as orc


@pytest.mark.parametrize("k", range(1, 9))
def test_c_ordered_strides_equal_numpy_indexing(k):
    rng = np.random.default_rng(k)
    batch = 50
    dims = [int(d) for d in rng.integers(1, 6, k)]
    shape = [batch] + dims
    W = rng.normal(0, 1, shape).astype(np.float32)
    strides = [int(np.prod(dims[i + 1:], dtype=np.int64)) for i in range(k)]
    idx = np.stack([rng.integers(0, d, batch) for d in dims], 1).astype(np.int32)
    got = orc.batch_gather(W, idx, strides, int(np.prod(dims)))
    want = W[(np.arange(batch),) + tuple(idx[:, i] for i in range(k))]
    assert np.array_equal(got, want)


def test_reference_three_index_case():
    w = np.arange(120, dtype=np.float32)
    got = orc.batch_gather(w, [[0, 1, 2], [1, 0, 3]], [60, 20, 1], 60)
    assert got.tolist() == [22.0, 0.0]


def test_u32_wrapping():
    """Random int32 indices, u32 strides and batch stride; the last stride is
    odd, so the last index can be solved for a target: every other row is
    steered into range (target < n_w) through wrapped negative products."""
    rng = np.random.default_rng(3)
    n_w = 1 << 12
    w = np.arange(n_w, dtype=np.float32) + 1000.0  # in range: lin + 1000, never 0
    batch, k = 400, 3
    M = 1 << 32
    idx = rng.integers(-(1 << 31), 1 << 31, (batch, k)).astype(np.int64)
    strides = [int(s) for s in rng.integers(0, M, k, dtype=np.uint64)]
    strides[-1] |= 1
    inv = pow(strides[-1], -1, M)
    bs = int(rng.integers(0, M, dtype=np.uint64))
    for b in range(0, batch, 2):
        part = (b * bs + sum((int(idx[b, i]) % M) * strides[i] for i in range(k - 1))) % M
        target = int(rng.integers(0, n_w))
        v = ((target - part) * inv) % M
        idx[b, -1] = v - M if v >= (1 << 31) else v
    idx = idx.astype(np.int32)
    got = orc.batch_gather(w, idx, strides, bs)
    inside = 0
    for b in range(batch):
        lin = (b * bs + sum((int(idx[b, i]) % M) * strides[i] for i in range(k))) % M
        assert got[b] == (lin + 1000.0 if lin < n_w else 0.0)
        inside += lin < n_w
    assert inside >= batch // 2
    # batch stride 1, stride 1: -1 wraps to 2^32 - 1 (out of range), then to 0
    got = orc.batch_gather(w, [[-1], [-1], [5]], [1], 1)
    assert got.tolist() == [0.0, 1000.0, 1007.0]
