"""The decision arithmetic: exp / sigmoid / log / Gumbel and the word threshold.

Pins (the reference's Burn sigmoid/log are not vendored, so the build defines
its own; spin_gibbs.rs:95-97, softmax.rs:86-93):
  - error bounds against float64 libm (exp 2 ulp, log and sigmoid 3 ulp);
  - identities: sigmoid(0) = 1/2, sigmoid(x) + sigmoid(-x) ~ 1, monotone;
  - Gumbel draws: mean = Euler-Mascheroni, variance = pi^2/6;
  - the oracle and the product header (host build) agree bit for bit;
  - word_threshold(p) reproduces `u <= p` for every tested (word, p);
  - the full-range forms (kernel-level exports): equal to the bounded forms
    on their ranges, error bounds against float64 libm down to subnormal
    results and inputs, and the IEEE limits at 0, 1, inf and NaN;
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
    L = ctypes.CDLL(os.path.join(HERE, "native", os.environ.get("THRML_NATIVE_BUILD", "build"),
                                "libproductshim.so"))
    f32p = ctypes.POINTER(ctypes.c_float)
    u32p = ctypes.POINTER(ctypes.c_uint32)
    for n in ("shim_exp", "shim_sigmoid", "shim_log", "shim_exp_full", "shim_sigmoid_full",
              "shim_log_full"):
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


def _special_inputs():
    f = np.float32
    return np.array([0.0, -0.0, 1.0, np.inf, -np.inf, np.nan, -1.0, 2.0**-149, 2.0**-140,
                     2.0**-126, 2.0**-127, 3 * 2.0**-149, 1 - 2.0**-24, 1e-45, 1e38, -1e38],
                    dtype=f)


def test_full_range_equal_bounded_forms_on_their_ranges():
    x = np.linspace(-80, 80, 400_001, dtype=np.float32)
    assert np.array_equal(orc.map_f32("exp_full", x).view(np.uint32),
                          orc.map_f32("exp", x).view(np.uint32))
    assert np.array_equal(orc.map_f32("sigmoid_full", x).view(np.uint32),
                          orc.map_f32("sigmoid", x).view(np.uint32))
    xl = np.geomspace(2.0**-126, 2.0**100, 400_001).astype(np.float32)
    assert np.array_equal(orc.map_f32("log_full", xl).view(np.uint32),
                          orc.map_f32("log", xl).view(np.uint32))


def test_full_range_error_bounds_and_limits():
    # exp over the whole finite range, subnormal and near-overflow results
    x = np.concatenate([np.linspace(-110, 90, 400_001),
                        np.linspace(-104, -87, 100_001)]).astype(np.float32)
    y = orc.map_f32("exp_full", x).astype(np.float64)
    want = np.exp(x.astype(np.float64))
    with np.errstate(over="ignore"):
        want32 = want.astype(np.float32)  # correctly rounded (double -> float)
    ulp = np.spacing(want32).astype(np.float64)
    fin = np.isfinite(want32)
    assert (np.abs(y[fin] - want[fin]) / ulp[fin]).max() <= 2.0
    assert np.all(np.isinf(y[~fin]))
    # sigmoid: 1/(1+exp(-x)) including results below the normal range; past
    # x = -88.72 the formula's exp(-x) overflows and the result is exactly 0,
    # as the reference's literal formula gives in IEEE arithmetic
    xs = np.linspace(-88.7, 100, 400_001).astype(np.float32)
    ys = orc.map_f32("sigmoid_full", xs).astype(np.float64)
    ws = 1.0 / (1.0 + np.exp(-xs.astype(np.float64)))
    us = np.spacing(ws.astype(np.float32)).astype(np.float64)
    assert (np.abs(ys - ws) / us).max() <= 3.0
    assert not orc.map_f32("sigmoid_full", np.linspace(-120, -88.8, 1000, dtype=np.float32)).any()
    # log of subnormal inputs (their true exponent) and of large ones
    xl = np.concatenate([np.geomspace(2.0**-149, 2.0**-126, 200_000),
                         np.geomspace(1e30, 3e38, 1000)]).astype(np.float32)
    yl = orc.map_f32("log_full", xl).astype(np.float64)
    wl = np.log(xl.astype(np.float64))
    assert (np.abs(yl - wl) / np.spacing(np.abs(wl).astype(np.float32))).max() <= 3.0
    # IEEE limits
    s = _special_inputs()
    ls = orc.map_f32("log_full", s)
    for v, r in zip(s, ls):
        if np.isnan(v) or v < 0:
            assert np.isnan(r), v
        elif v == 0:
            assert r == -np.inf
        elif v == np.inf:
            assert r == np.inf
        elif v == 1.0:
            assert r == 0.0
    e = orc.map_f32("exp_full", np.array([-np.inf, -200, -104.5, np.inf, 200, np.nan], np.float32))
    assert e[0] == 0 and e[1] == 0 and e[2] == 0 and e[3] == np.inf and e[4] == np.inf
    assert np.isnan(e[5])
    sg = orc.map_f32("sigmoid_full", np.array([-200, -88, 200, np.nan], np.float32))
    assert sg[0] == 0.0 and 0.0 < sg[1] < 2.0**-126 and sg[2] == 1.0 and np.isnan(sg[3])


def test_product_full_range_matches_oracle_bitwise(shim):
    rng = np.random.default_rng(9)
    x = np.concatenate([np.linspace(-120, 120, 300_001), rng.normal(0, 40, 100_000),
                        _special_inputs()]).astype(np.float32)
    xl = np.concatenate([np.abs(x), np.geomspace(2.0**-149, 1.0, 100_000).astype(np.float32),
                         _special_inputs()]).astype(np.float32)
    for name, sname, arg in (("exp_full", "shim_exp_full", x),
                             ("sigmoid_full", "shim_sigmoid_full", x),
                             ("log_full", "shim_log_full", xl)):
        a = orc.map_f32(name, arg)
        b = _call(getattr(shim, sname), arg)
        same = (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))
        assert same.all(), name


def test_gumbel_argmax_restatement_rules():
    """The reference kernel's rules that hold whatever the log's rounding:
    exact ties (equal logit and uniform) give the first index; u = 0 scores
    -inf and is never taken after index 0; u = 1 scores +inf and is taken
    (the first such column); a NaN score never wins after index 0
    (gumbel_argmax/kernel.rs:59-83)."""
    q = 6
    rng = np.random.default_rng(4)
    n = 4000
    L = rng.normal(0, 1, (n, q)).astype(np.float32)
    U = rng.uniform(0.01, 0.99, (n, q)).astype(np.float32)
    # ties: copy column a into b > a in each row
    a = rng.integers(0, q - 1, n)
    b = a + 1 + rng.integers(0, q - 1 - a)
    L[np.arange(n), b] = L[np.arange(n), a]
    U[np.arange(n), b] = U[np.arange(n), a]
    # make the tied pair the clear winner
    L[np.arange(n), a] += 50.0
    L[np.arange(n), b] += 50.0
    got = orc.gumbel_argmax(L, U)
    assert np.array_equal(got, a)
    # u = 0: never chosen past index 0, even with the largest logit
    L2 = rng.normal(0, 1, (n, q)).astype(np.float32)
    U2 = rng.uniform(0.01, 0.99, (n, q)).astype(np.float32)
    z = rng.integers(1, q, n)
    L2[np.arange(n), z] = 100.0
    U2[np.arange(n), z] = 0.0
    assert not np.any(orc.gumbel_argmax(L2, U2) == z)
    # u = 1: +inf score, the first such column wins
    U3 = U2.copy()
    U3[np.arange(n), z] = 1.0
    L3 = L2.copy()
    L3[np.arange(n), z] = -100.0
    got3 = orc.gumbel_argmax(L3, U3)
    assert np.array_equal(got3, z)
    # NaN uniform (or u > 1) in a later column never wins; index 0 NaN sticks
    U4 = U2.copy()
    U4[:, 1] = np.nan
    L4 = L2.copy()
    L4[:, 1] = 1000.0
    assert not np.any(orc.gumbel_argmax(L4, U4) == 1)
    U5 = np.full((3, q), 0.5, np.float32)
    U5[:, 0] = np.nan
    assert np.array_equal(orc.gumbel_argmax(np.zeros((3, q), np.float32), U5), [0, 0, 0])


def test_sigmoid_bernoulli_restatement_limits():
    """u < sigmoid(2 gamma), strict (sigmoid_bernoulli/kernel.rs:53): u = 0
    samples 0 once exp(-2 gamma) overflows and the probability is 0 (2 gamma
    below -88.72), and 1 wherever it is positive, subnormal included."""
    g = np.array([-60.0, -44.3, -30.0, 0.0, 40.0, 60.0], np.float32)
    u0 = np.zeros_like(g)
    assert np.array_equal(orc.sigmoid_bernoulli(g, u0), [0, 1, 1, 1, 1, 1])
    u1 = np.full_like(g, np.float32(1 - 2.0**-24))
    assert np.array_equal(orc.sigmoid_bernoulli(g, u1), [0, 0, 0, 0, 1, 1])
    assert np.array_equal(orc.sigmoid_bernoulli(g, np.full_like(g, 0.5)), [0, 0, 0, 0, 1, 1])
