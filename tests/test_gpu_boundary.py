"""The C ABI's edges on the GPU: the kernel-level exports at IEEE corner
inputs (planted ties, u = 0, u = 1, subnormal and NaN uniforms, extreme
pre-activations) against the oracle's restatement of the reference kernels
(crates/thrml-kernels/src/gumbel_argmax/kernel.rs:47-88,
crates/thrml-kernels/src/sigmoid_bernoulli/kernel.rs:34-55), and the batch
gather export (batch_gather/kernel.rs) with wrapping and out-of-range
indices; rejection of
out-of-range state values from host and device memory; contexts created and
destroyed on several threads while other threads run sweeps."""
import ctypes
import threading

import numpy as np
import pytest

import pyoracle as orc
import thrml_hip as th
from conftest import log_case
from thrml_hip import _lib
from thrml_hip import workloads as wl

pytestmark = pytest.mark.gpu


def _gumbel_export(device, logits, u):
    import torch

    n, q = logits.shape
    ld = torch.from_numpy(np.ascontiguousarray(logits)).cuda()
    ud = torch.from_numpy(np.ascontiguousarray(u)).cuda()
    od = torch.empty(n, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    _lib.check(_lib.load().thrml_gumbel_argmax(device.handle, ctypes.c_void_p(ld.data_ptr()),
                                               ctypes.c_void_p(ud.data_ptr()),
                                               ctypes.c_void_p(od.data_ptr()), n, q))
    device.synchronize()
    return od.cpu().numpy()


def _bernoulli_export(device, gamma, u):
    import torch

    gd = torch.from_numpy(np.ascontiguousarray(gamma)).cuda()
    ud = torch.from_numpy(np.ascontiguousarray(u)).cuda()
    od = torch.empty(gamma.size, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    _lib.check(_lib.load().thrml_sigmoid_bernoulli(device.handle, ctypes.c_void_p(gd.data_ptr()),
                                                   ctypes.c_void_p(ud.data_ptr()),
                                                   ctypes.c_void_p(od.data_ptr()), gamma.size))
    device.synchronize()
    return od.cpu().numpy()


def test_gumbel_export_planted_ties_and_limits(device):
    log_case("gumbel export: ties, u=0, u=1, subnormal, NaN")
    rng = np.random.default_rng(21)
    n, q = 8192, 8
    L = rng.normal(0, 1, (n, q)).astype(np.float32)
    U = rng.uniform(0.0, 1.0, (n, q)).astype(np.float32)
    r = np.arange(n)
    kind = r % 6
    a = rng.integers(0, q - 1, n)
    b = a + 1 + rng.integers(0, q - 1 - a)
    # 0: exact tie of two columns as the clear winner -> first of them
    m = kind == 0
    L[m, b[m]] = L[m, a[m]] = 40.0
    U[m, b[m]] = U[m, a[m]]
    # 1: u = 0 on the largest logit -> never taken (score -inf)
    m = kind == 1
    L[m, b[m]] = 100.0
    U[m, b[m]] = 0.0
    # 2: u = 1 on two columns -> the first of them (score +inf)
    m = kind == 2
    U[m, a[m]] = 1.0
    U[m, b[m]] = 1.0
    # 3: subnormal uniforms (finite, very negative log) and -0.0
    m = kind == 3
    U[m, a[m]] = np.float32(3 * 2.0**-149)
    U[m, b[m]] = -0.0
    # 4: NaN and u > 1 in later columns, a huge logit there
    m = kind == 4
    U[m, b[m]] = np.nan
    L[m, b[m]] = 1e30
    U[m, a[m]] = 1.5
    # 5: plain random rows
    got = _gumbel_export(device, L, U)
    want = orc.gumbel_argmax(L, U)
    assert np.array_equal(got, want)
    # the rules themselves, whatever the log's rounding
    assert np.array_equal(got[kind == 0], a[kind == 0])
    assert not np.any(got[kind == 1] == b[kind == 1])
    assert np.array_equal(got[kind == 2], a[kind == 2])
    assert not np.any(got[kind == 4] == b[kind == 4])


def test_sigmoid_bernoulli_export_limits(device):
    log_case("sigmoid-bernoulli export: extreme pre-activations, u = 0")
    rng = np.random.default_rng(22)
    g = np.concatenate([rng.normal(0, 30, 20000), np.linspace(-60, 60, 20001),
                        [-1e30, -44.3, -44.4, 0.0, 1e30, np.nan]]).astype(np.float32)
    for u in (np.zeros_like(g), rng.random(g.size).astype(np.float32),
              np.full_like(g, np.float32(1 - 2.0**-24)),
              np.full_like(g, np.float32(2.0**-140))):
        got = _bernoulli_export(device, g, u)
        assert np.array_equal(got, orc.sigmoid_bernoulli(g, u))
    # u = 0 with a vanishing probability samples 0 (sigmoid underflows to 0)
    assert _bernoulli_export(device, np.array([-60.0], np.float32), np.zeros(1, np.float32))[0] == 0


def test_state_rejects_out_of_range_values(device):
    import torch

    log_case("state import: out-of-range spins and categories")
    ebm, blocks = wl.lattice_ising(8, 0.1, 0.3, 0.05)
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    st = prog.new_state(5)
    good = np.random.default_rng(0).integers(0, 2, (5, 32)).astype(np.uint8)
    st.set_block(0, good)
    for dtype, badval in ((np.uint8, 2), (np.uint8, 255), (np.float32, 0.5),
                          (np.float32, np.nan), (np.float32, -1.0)):
        bad = 1 - good.astype(dtype)
        bad[4, 31] = badval
        with pytest.raises(th.ThrmlError, match="spin value out of range"):
            st.set_block(0, bad)
        with pytest.raises(th.ThrmlError, match="spin value out of range"):
            st.set_block(0, torch.from_numpy(bad).cuda())
        # a rejected import writes nothing: the block keeps its values
        assert np.array_equal(st.get_block(0), good)
    st.set_block(0, good)  # the state stays usable
    assert np.array_equal(st.get_block(0), good)

    q = 5
    n, edges, W, bias, pblocks = wl.potts_lattice(8, q, 0.5, 0.3, cfg=9)
    cp = th.CategoricalProgram(n, q, edges, W, bias, pblocks, device)
    cs = cp.new_state(7)
    nb = cp.block_range(0)[1]
    good = np.random.default_rng(1).integers(0, q, (7, nb)).astype(np.uint8)
    cs.set_block(0, good)
    for badval in (q, 255):
        bad = (q - 1 - good).astype(np.uint8)
        bad[3, 5] = badval
        with pytest.raises(th.ThrmlError, match="category value out of range"):
            cs.set_block(0, bad)
        with pytest.raises(th.ThrmlError, match="category value out of range"):
            cs.set_block(0, torch.from_numpy(bad).cuda())
        assert np.array_equal(cs.get_block(0), good)
    for badval in (-1.0, 1.5, float(q), np.nan, np.inf):
        bad = good.astype(np.float32)
        bad[6, 0] = badval
        with pytest.raises(th.ThrmlError, match="category value out of range"):
            cs.set_block(0, bad)
    # integer and float64 input that a byte cannot hold is rejected, not wrapped
    # (256 + 2 would read as category 2, -255 as 1)
    for dtype, badval in ((np.int64, 256 + 2), (np.int32, -255), (np.uint16, 261),
                          (np.float64, 2.5), (np.float64, 1e10)):
        bad = good.astype(dtype)
        bad[2, 2] = badval
        with pytest.raises(th.ThrmlError, match="category value out of range"):
            cs.set_block(0, bad)
        assert np.array_equal(cs.get_block(0), good)
    cs.set_block(0, good.astype(np.int64))
    cs.set_block(0, good.astype(np.float32))
    assert np.array_equal(cs.get_block(0), good)
    th.run_blocks(th.RngKey(3), cp, cs, (), 2)  # a sweep after the rejections runs normally
    assert cs.get_global().max() < q


def test_contexts_created_and_destroyed_across_threads():
    """Context creation and destruction on some threads while others run
    sweeps and moment runs on their own contexts: the results equal those of
    a single-threaded run."""
    log_case("contexts across threads")
    ebm, blocks = wl.lattice_ising(32, 0.1, 0.4, 0.05)
    ref_dev = th.Device(0)
    ref_prog = th.IsingSamplingProgram(ebm, blocks, [], ref_dev)
    st = th.hinton_init(th.RngKey(1), ref_prog, 64)
    init = st.get_global()
    th.run_blocks(th.RngKey(2), ref_prog, st, (), 20)
    want = st.get_global()
    errors, results = [], []

    def runner(k):
        try:
            dev = th.Device(0)
            prog = th.IsingSamplingProgram(ebm, blocks, [], dev)
            for _ in range(5):
                s = prog.new_state(64)
                s.set_global(init)
                th.run_blocks(th.RngKey(2), prog, s, (), 20)
                results.append(np.array_equal(s.get_global(), want))
                s.close()
            prog.close()
            dev.close()
        except Exception as e:  # reported below
            errors.append(repr(e))

    def churner():
        try:
            for _ in range(40):
                d = th.Device(0)
                d.close()
        except Exception as e:
            errors.append(repr(e))

    threads = [threading.Thread(target=runner, args=(k,)) for k in range(4)]
    threads += [threading.Thread(target=churner) for _ in range(3)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads)
    assert not errors, errors
    assert len(results) == 20 and all(results)
    # closing the context first also closes the state and program made on it
    ref_dev.close()
    assert not st._h.value and not ref_prog._h.value


def _gather_export(device, weights, indices, strides, batch_stride):
    import torch

    wd = torch.from_numpy(np.ascontiguousarray(np.asarray(weights, np.float32).reshape(-1))).cuda()
    idx = np.ascontiguousarray(np.asarray(indices, np.int32))
    idx = idx.reshape(idx.shape[0], idx.shape[1] if idx.ndim > 1 else 1)
    idd = torch.from_numpy(idx).cuda()
    st = np.ascontiguousarray(np.asarray(strides, np.uint32))
    od = torch.empty(idx.shape[0], dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    _lib.check(_lib.load().thrml_batch_gather(
        device.handle, ctypes.c_void_p(wd.data_ptr()), wd.numel(), ctypes.c_void_p(idd.data_ptr()),
        idx.shape[0], idx.shape[1], st.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
        int(batch_stride), ctypes.c_void_p(od.data_ptr())))
    device.synchronize()
    return od.cpu().numpy()


@pytest.mark.parametrize("k", [1, 2, 3, 5, 8, 64])
def test_batch_gather_export(device, k):
    """thrml_batch_gather (batch_gather_fused) against the oracle, bit for bit:
    C-ordered strides with in-range indices, then random int32 indices with
    u32 strides (wrapping, mostly out of range: 0.0), 1M rows."""
    log_case(f"batch_gather export k={k}")
    rng = np.random.default_rng(100 + k)
    batch = 1 << 20
    dims = [1] * (k - 8) + [2] * 8 if k > 8 else [int(d) for d in rng.integers(1, 5, k)]
    n = int(np.prod(dims))
    W = rng.normal(0, 1, (min(batch, 4096), n)).astype(np.float32)
    strides = [int(np.prod(dims[i + 1:], dtype=np.int64)) for i in range(k)]
    idx = np.stack([rng.integers(0, d, batch) for d in dims], 1).astype(np.int32)
    for bs in (n, 0):
        got = _gather_export(device, W, idx, strides, bs)
        assert np.array_equal(got, orc.batch_gather(W, idx, strides, bs))
    idx = rng.integers(-(1 << 31), 1 << 31, (batch, k)).astype(np.int32)
    st = rng.integers(0, 1 << 32, k, dtype=np.uint64)
    got = _gather_export(device, W, idx, st, 7)
    assert np.array_equal(got, orc.batch_gather(W, idx, st, 7))


def test_batch_gather_export_checks(device):
    with pytest.raises(th.ThrmlError, match="at most 64 indices"):
        _gather_export(device, np.zeros(4), np.zeros((2, 65)), np.zeros(65), 1)
    assert _gather_export(device, np.arange(4.0), np.zeros((0, 2)), [1, 1], 1).size == 0
