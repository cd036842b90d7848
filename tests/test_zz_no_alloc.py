"""thrml_run_blocks_noalloc (no counterpart in the reference: run_blocks for
callers that cannot allocate) against thrml_run_blocks, through the C ABI:
identical states on two calls in a row, the second with a smaller input;
a run long enough to need several chunks of the fixed key array; the
rejection of a state whose one sweep needs more key bytes than the array,
and of a context with kernel timing on; two contexts on one GPU (two
streams) whose calls are queued back to back without a host wait: the
second call's key schedule would overwrite keys the first call's sweeps
still read, unless the library orders them on the GPU."""
import numpy as np
import pytest

import thrml_hip as th
from conftest import log_case
from thrml_hip import _lib
from thrml_hip import workloads as wl

pytestmark = pytest.mark.gpu

KEY_WORDS_BYTES = 96  # expanded ChaCha8 key per (sweep, block, chain)
NOALLOC_BYTES = 16 << 20


def _noalloc(prog, key, st, n):
    _lib.check(_lib.load().thrml_run_blocks_noalloc(prog._h, key.seed, st._h, int(n)))


def _pair(prog, C, init, key, n):
    """(noalloc result, run_blocks result) from the same initial state."""
    a = prog.new_state(C)
    a.set_global(init)
    b = prog.new_state(C)
    b.set_global(init)
    _noalloc(prog, key, a, n)
    th.run_blocks(key, prog, b, (), n)
    out = a.get_global(), b.get_global()
    a.close()
    b.close()
    return out


def test_noalloc_equals_run_blocks_two_calls(device):
    rng = np.random.default_rng(17)
    # first call: lattice program, 4096 chains; one sweep needs 2 x 4096 x 96
    # = 786 KiB of keys, so 50 sweeps take three chunks of the 16 MiB array
    ebm, blocks = wl.lattice_ising(32, 0.1, 0.4, 0.05)
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    assert prog.kind == "lattice"
    C = 4096
    assert 2 * C * KEY_WORDS_BYTES * 50 > 2 * NOALLOC_BYTES
    init = rng.integers(0, 2, (C, ebm.n_nodes)).astype(np.uint8)
    log_case("noalloc call 1: lattice 32^2, 4096 chains, 50 sweeps")
    got, want = _pair(prog, C, init, th.RngKey(5), 50)
    assert np.array_equal(got, want)
    # second call, smaller: a CSR program (side 10 is not a multiple of 32),
    # 37 chains, 7 sweeps (the array keeps the first call's larger contents)
    ebm2, blocks2 = wl.lattice_ising(10, 0.3, 0.2, 0.5)
    prog2 = th.IsingSamplingProgram(ebm2, blocks2, [], device)
    assert prog2.kind == "csr"
    init2 = rng.integers(0, 2, (37, ebm2.n_nodes)).astype(np.uint8)
    log_case("noalloc call 2: CSR 10^2, 37 chains, 7 sweeps")
    got2, want2 = _pair(prog2, 37, init2, th.RngKey(6), 7)
    assert np.array_equal(got2, want2)
    # and once more at the first size: no state carried over between calls
    log_case("noalloc call 3: lattice again")
    got3, want3 = _pair(prog, C, init, th.RngKey(5), 50)
    assert np.array_equal(got3, want3) and np.array_equal(got3, got)


def test_noalloc_categorical_and_dense(device):
    rng = np.random.default_rng(18)
    n, edges, W, bias, blocks = wl.potts_lattice(16, 4, 0.5, 0.3, cfg=9)
    prog = th.CategoricalProgram(n, 4, edges, W, bias, blocks, device)
    init = rng.integers(0, 4, (70, n)).astype(np.uint8)
    log_case("noalloc categorical 16^2 q=4, 70 chains")
    got, want = _pair(prog, 70, init, th.RngKey(8), 6)
    assert np.array_equal(got, want)
    bits, _ = th.bf16_round(rng.normal(0, 0.1, (100, 60)).astype(np.float32))
    rp = th.RbmProgram(bits, rng.normal(0, 0.2, 100), rng.normal(0, 0.2, 60), 1.0, device)
    init = rng.integers(0, 2, (300, 160)).astype(np.uint8)
    log_case("noalloc dense 100 x 60, 300 chains")
    got, want = _pair(rp, 300, init, th.RngKey(9), 4)
    assert np.array_equal(got, want)


def test_noalloc_rejects_oversized_and_timed(device):
    # 10 colour blocks x 300 chain groups: 10 x 19200 x 96 bytes per sweep > 16 MiB
    edges = np.array([(i, i + 1) for i in range(19)], np.uint32)
    ebm = th.IsingEBM(20, edges, np.zeros(20, np.float32), np.ones(19, np.float32))
    blocks = [th.Block([2 * k, 2 * k + 1]) for k in range(10)]
    prog = th.IsingSamplingProgram(ebm, blocks, [], device)
    C = 64 * 300
    assert 10 * C * KEY_WORDS_BYTES > NOALLOC_BYTES
    st = prog.new_state(C)
    log_case("noalloc oversized state is rejected")
    with pytest.raises(th.ThrmlError, match="THRML_NOALLOC_KEY_BYTES"):
        _noalloc(prog, th.RngKey(1), st, 1)
    st.close()
    small = prog.new_state(64)
    device.enable_timing(True)
    try:
        with pytest.raises(th.ThrmlError, match="timing"):
            _noalloc(prog, th.RngKey(1), small, 1)
    finally:
        device.enable_timing(False)
    _noalloc(prog, th.RngKey(1), small, 3)  # accepted once timing is off


def test_noalloc_two_contexts_share_the_key_array(device):
    rng = np.random.default_rng(19)
    dev_b = th.Device(0)  # a second context: its own stream on the same GPU
    try:
        ebm, blocks = wl.lattice_ising(64, 0.1, 0.4, 0.05)
        prog_a = th.IsingSamplingProgram(ebm, blocks, [], device)
        ebm2, blocks2 = wl.lattice_ising(10, 0.3, 0.2, 0.5)
        prog_b = th.IsingSamplingProgram(ebm2, blocks2, [], dev_b)
        Ca, Cb = 2048, 100
        init_a = rng.integers(0, 2, (Ca, ebm.n_nodes)).astype(np.uint8)
        init_b = rng.integers(0, 2, (Cb, ebm2.n_nodes)).astype(np.uint8)
        # the expected results, each context on its own
        want_a = prog_a.new_state(Ca)
        want_a.set_global(init_a)
        th.run_blocks(th.RngKey(31), prog_a, want_a, (), 100)
        want_b = prog_b.new_state(Cb)
        want_b.set_global(init_b)
        th.run_blocks(th.RngKey(32), prog_b, want_b, (), 9)
        for rep in range(3):
            log_case(f"noalloc from two contexts back to back, repeat {rep}")
            a = prog_a.new_state(Ca)
            a.set_global(init_a)
            b = prog_b.new_state(Cb)
            b.set_global(init_b)
            device.synchronize()
            dev_b.synchronize()
            # queued without a host wait in between: 100 sweeps of 2048 chains
            # (one sweep needs 2 x 2048 x 96 bytes of keys: three chunks of
            # the array, each key schedule rewriting it from the start), then
            # a short run on the other stream
            assert 100 * 2 * Ca * KEY_WORDS_BYTES > 2 * NOALLOC_BYTES
            _noalloc(prog_a, th.RngKey(31), a, 100)
            _noalloc(prog_b, th.RngKey(32), b, 9)
            got_b = b.get_global()
            got_a = a.get_global()
            assert np.array_equal(got_b, want_b.get_global())
            assert np.array_equal(got_a, want_a.get_global())
            a.close()
            b.close()
    finally:
        dev_b.close()
