"""RngKey splitting and the ChaCha8 keystream (crates/thrml-samplers/src/rng.rs).

Pins: RFC 8439 block vectors (20 rounds), the published ChaCha8 zero-key
keystream, rand_core 0.6's seed_from_u64(0) constant; the reference's own
rng.rs:57-86 tests (uniqueness, determinism); and agreement of three
implementations (oracle C, product header on the host, product C ABI).
"""
import ctypes
import json
import os

import numpy as np
import pytest

import pyoracle as orc

HERE = os.path.dirname(os.path.abspath(__file__))
VEC = json.load(open(os.path.join(HERE, "golden", "chacha_vectors.json")))


def _shim():
    import subprocess

    subprocess.run(["make", "-s", "-C", os.path.join(HERE, "native")], check=True)
    L = ctypes.CDLL(os.path.join(HERE, "native", os.environ.get("THRML_NATIVE_BUILD", "build"),
                                "libproductshim.so"))
    u32p = ctypes.POINTER(ctypes.c_uint32)
    L.shim_chacha_rfc.argtypes = [u32p, ctypes.c_int] + [ctypes.c_uint32] * 4 + [u32p]
    L.shim_chacha8.argtypes = [u32p, ctypes.c_uint64, u32p]
    L.shim_chacha8_pre.argtypes = [u32p, ctypes.c_uint32, u32p]
    L.shim_seed.argtypes = [ctypes.c_uint64, u32p]
    L.shim_split_at.argtypes = [ctypes.c_uint64] * 3
    L.shim_split_at.restype = ctypes.c_uint64
    L.shim_stream_word.argtypes = [u32p, ctypes.c_uint64]
    L.shim_stream_word.restype = ctypes.c_uint32
    return L


@pytest.fixture(scope="module")
def shim():
    return _shim()


def _key_words(key_bytes):
    b = bytes(key_bytes)
    return np.frombuffer(b, dtype="<u4").astype(np.uint32)


def _p(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))


def test_rfc8439_block_oracle():
    v = VEC["rfc8439_2_3_2"]
    k = _key_words(v["key"])
    out = orc.chacha_block(k, v["w12"] | (v["w13"] << 32), v["w14"] | (v["w15"] << 32), rounds=20)
    assert [f"{w:08x}" for w in out] == v["out"]
    v = VEC["rfc8439_a1_1"]
    out = orc.chacha_block(_key_words(v["key"]), 0, 0, rounds=20)
    assert [f"{w:08x}" for w in out] == v["out"]


def test_rfc8439_block_product(shim):
    v = VEC["rfc8439_2_3_2"]
    k = np.ascontiguousarray(_key_words(v["key"]))
    out = np.zeros(16, np.uint32)
    shim.shim_chacha_rfc(_p(k), 20, v["w12"], v["w13"], v["w14"], v["w15"], _p(out))
    assert [f"{w:08x}" for w in out] == v["out"]


def test_chacha8_zero_key_vector(shim):
    v = VEC["chacha8_zero"]
    want = bytes.fromhex(v["bytes"])
    out = orc.chacha_block(np.zeros(8, np.uint32), 0, 0, rounds=8)
    assert out.astype("<u4").tobytes() == want
    k = np.zeros(8, np.uint32)
    o2 = np.zeros(16, np.uint32)
    shim.shim_chacha8(_p(k), 0, _p(o2))
    assert o2.astype("<u4").tobytes() == want


def test_seed_from_u64_constant(shim):
    k = orc.seed_from_u64(0)
    assert int(k[0]) | (int(k[1]) << 32) == VEC["seed_from_u64_0"]
    k2 = np.zeros(8, np.uint32)
    for s in [0, 1, 42, 2**63 + 5, 2**64 - 1]:
        shim.shim_seed(s, _p(k2))
        assert np.array_equal(k2, orc.seed_from_u64(s))


def test_split_semantics():
    # rng.rs:20-27: n=0 -> [], n=1 -> [self]
    assert orc.rng_split(42, 0) == []
    assert orc.rng_split(42, 1) == [42]
    # rng.rs:57-70: 5 keys, all distinct
    ks = orc.rng_split(42, 5)
    assert len(set(ks)) == 5
    # rng.rs:72-85: deterministic
    assert orc.rng_split(42, 10) == orc.rng_split(42, 10)
    # prefix property of a sequential stream: split(n)[i] does not depend on n>=2
    assert orc.rng_split(42, 10)[:5] == ks


def test_split_first_key_is_first_u64_of_stream():
    # next_u64 = w[0] | w[1] << 32 of block 0 of ChaCha8(seed_from_u64(key))
    k8 = orc.seed_from_u64(7)
    blk = orc.chacha_block(k8, 0, 0, rounds=8)
    assert orc.rng_split(7, 3)[0] == int(blk[0]) | (int(blk[1]) << 32)
    assert orc.rng_split(7, 3)[2] == int(blk[4]) | (int(blk[5]) << 32)
    # element 8 lives in block 1
    blk1 = orc.chacha_block(k8, 1, 0, rounds=8)
    assert orc.rng_split(7, 9)[8] == int(blk1[0]) | (int(blk1[1]) << 32)


def test_product_split_matches_oracle(shim):
    import thrml_hip

    rng = np.random.default_rng(1)
    for key in [0, 1, 42, 2**64 - 1] + [int(x) for x in rng.integers(0, 2**63, 20)]:
        for n in [0, 1, 2, 3, 8, 9, 17, 100]:
            want = orc.rng_split(key, n)
            got = [k.seed for k in thrml_hip.RngKey(key).split(n)]
            assert got == want
            for i in range(n):
                assert shim.shim_split_at(key, n, i) == want[i]


def test_stream_word_counter_based(shim):
    k8 = np.ascontiguousarray(orc.seed_from_u64(99))
    for w in [0, 1, 15, 16, 31, 1000, 2**20 + 3]:
        assert shim.shim_stream_word(_p(k8), w) == orc.stream_word(k8, w)


def test_expanded_key_block_equals_oracle_block(shim):
    """The sweep kernels' ChaCha8 from a pre-expanded key (the key-only
    column quarter rounds and diagonal steps of the first double round
    computed once) gives the oracle's block for every counter below 2^32,
    including the extremes."""
    rng = np.random.default_rng(11)
    for _ in range(200):
        k = rng.integers(0, 2**32, 8, dtype=np.uint64).astype(np.uint32)
        for ctr in (0, 1, int(rng.integers(0, 2**32)), 2**32 - 1):
            a = np.zeros(16, np.uint32)
            shim.shim_chacha8_pre(_p(k), ctr, _p(a))
            assert np.array_equal(a, orc.chacha_block(k, ctr))
