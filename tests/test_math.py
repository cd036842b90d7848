"""The decision arithmetic: exp / sigmoid / log / Gumbel and the word threshold.

Pins (the reference's Burn sigmoid/log are not vendored, so the build defines
its own; spin_gibbs.rs:95-97, softmax.rs:86-93):
  - error bounds against float64 libm (exp 2 ulp, log and sigmoid 3 ulp);
  - identities: sigmoid(0) = 1/2, sigmoid(x) + sigmoid(-x) ~ 1, monotone;
  - Gumbel draws: mean = Euler-Mascheroni, variance = pi^2/6;
  - the oracle and the product header (host build) agree bit for bit;
  - word_threshold(p) reproduces `u <= p` for every tested (word, p);
  - the kernels' index division by a launch constant (FastDiv) equals integer
    division for every divisor up to 4096, powers of two and their
    neighbours, and random divisors, at dividends up to 2^31 - 1.
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

import pyoracle as orc

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def shim():
    subprocess.run(["make", "-s", "-C", os.path.join(HERE, "native")], check=True)
    L = ctypes.CDLL(os.path.join(HERE, "native", "build", "libproductshim.so"))
    f32p = ctypes.POINTER(ctypes.c_float)
    u32p = ctypes.POINTER(ctypes.c_uint32)
    for n in ("shim_exp", "shim_sigmoid", "shim_log"):
        getattr(L, n).argtypes = [f32p, f32p, ctypes.c_uint64]
    L.shim_gumbel.argtypes = [u32p, f32p, ctypes.c_uint64]
    L.shim_threshold.argtypes = [f32p, u32p, ctypes.c_uint64]
    L.shim_fastdiv.argtypes = [ctypes.c_uint32, u32p, u32p, ctypes.c_uint64]
    return L


def _call(fn, x, out_dtype=np.float32, in_t=ctypes.c_float, out_t=ctypes.c_float):
    x = np.ascontiguousarray(x)
    y = np.zeros(x.shape, out_dtype)
    fn(x.ctypes.data_as(ctypes.POINTER(in_t)), y.ctypes.data_as(ctypes.POINTER(out_t)), x.size)
    return y


def _ulp_err(got, want):
    got = got.astype(np.float64)
    ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    return np.abs(got - want) / ulp


def test_exp_error_bound():
    x = np.linspace(-80, 80, 400_001, dtype=np.float32)
    y = orc.map_f32("exp", x)
    assert _ulp_err(y, np.exp(x.astype(np.float64))).max() <= 2.0


def test_sigmoid_error_bound_and_identities():
    x = np.linspace(-30, 30, 300_001, dtype=np.float32)
    y = orc.map_f32("sigmoid", x)
    want = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    assert _ulp_err(y, want).max() <= 3.0
    assert orc.sigmoid(0.0) == np.float32(0.5)
    assert np.all(np.diff(y.astype(np.float64)) >= 0)  # monotone
    assert np.abs(y + y[::-1] - 1.0).max() < 1e-6
    # clamp: saturates without denormals or NaN
    assert orc.sigmoid(1e30) == 1.0 and 0.0 < orc.sigmoid(-1e30) < 1e-34


def test_log_error_bound():
    x = np.concatenate([np.geomspace(1e-8, 100, 300_000), np.linspace(0.5, 2.0, 100_001)]).astype(np.float32)
    y = orc.map_f32("log", x)
    want = np.log(x.astype(np.float64))
    err = np.abs(y.astype(np.float64) - want)
    ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    # near x = 1 the result is tiny; bound absolute error by 2^-24 there
    assert np.all((err / ulp <= 3.0) | (err <= 2.0**-24))


def test_gumbel_moments():
    rng = np.random.default_rng(0)
    w = rng.integers(0, 2**32, 2_000_000, dtype=np.uint64).astype(np.uint32)
    g = orc.map_gumbel(w).astype(np.float64)
    assert np.isfinite(g).all()
    assert abs(g.mean() - 0.5772156649) < 5e-3
    assert abs(g.var() - np.pi**2 / 6) < 1e-2


def test_product_header_matches_oracle_bitwise(shim):
    rng = np.random.default_rng(3)
    x = np.concatenate([np.linspace(-90, 90, 200_001), rng.normal(0, 3, 200_000)]).astype(np.float32)
    for name, sname in (("exp", "shim_exp"), ("sigmoid", "shim_sigmoid")):
        xx = np.clip(x, -80, 80) if name == "exp" else x
        a = orc.map_f32(name, xx)
        b = _call(getattr(shim, sname), xx)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), name
    xl = np.abs(x) + np.float32(1e-6)
    a = orc.map_f32("log", xl)
    b = _call(shim.shim_log, xl)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    w = rng.integers(0, 2**32, 500_000, dtype=np.uint64).astype(np.uint32)
    a = orc.map_gumbel(w)
    b = _call(shim.shim_gumbel, w, in_t=ctypes.c_uint32)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_word_threshold_equals_uniform_compare(shim):
    rng = np.random.default_rng(5)
    p = np.concatenate([rng.random(20000), [0.0, 1.0, 2.0**-24, 1 - 2.0**-24, 0.5, 2.0**-30],
                        orc.map_f32("sigmoid", rng.normal(0, 6, 20000))]).astype(np.float32)
    t = _call(shim.shim_threshold, p, np.uint32, out_t=ctypes.c_uint32)
    for k in range(0, p.size, 97):
        words = np.concatenate([rng.integers(0, 2**32, 64, dtype=np.uint64).astype(np.uint32),
                                np.array([0, 255, 256, 2**32 - 1], np.uint32)])
        # candidate words right at the boundary of this p
        m = int(np.floor(np.float64(p[k]) * 2**24))
        for d in (-1, 0, 1):
            mm = min(max(m + d, 0), 2**24 - 1)
            words = np.append(words, np.array([(mm << 8), (mm << 8) | 255], np.uint32))
        u = (words >> 8).astype(np.float32) * np.float32(2.0**-24)
        assert np.array_equal(u <= p[k], words <= t[k]), (p[k], t[k])


def test_fastdiv_equals_integer_division(shim):
    rng = np.random.default_rng(11)
    divisors = set(range(1, 4097))
    for k in range(1, 31):
        divisors |= {2 ** k - 1, 2 ** k, 2 ** k + 1}
    divisors |= set(int(v) for v in rng.integers(1, 2 ** 31, 300))
    top = 2 ** 31 - 1
    base = np.concatenate([np.arange(0, 5000), np.arange(top - 5000, top + 1),
                           rng.integers(0, 2 ** 31, 20000)]).astype(np.uint32)
    for d in sorted(divisors):
        if d >= 2 ** 32:
            continue
        # multiples of d and their neighbours, where a rounding error would show
        mult = (np.arange(1, 200, dtype=np.uint64) * d)
        mult = np.concatenate([mult - 1, mult])
        mult = mult[mult <= top].astype(np.uint32)
        x = np.ascontiguousarray(np.concatenate([base, mult]))
        q = np.zeros_like(x)
        shim.shim_fastdiv(d, x.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                          q.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), x.size)
        assert np.array_equal(q, x // np.uint32(d)), d
