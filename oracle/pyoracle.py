"""ctypes binding of the CPU oracle (oracle/build/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the product package.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# THRML_ORACLE_BUILD=build-san selects the sanitizer build (make -C oracle san)
LIB_PATH = os.path.join(HERE, os.environ.get("THRML_ORACLE_BUILD", "build"), "liboracle.so")

_u32p = ctypes.POINTER(ctypes.c_uint32)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_i64p = ctypes.POINTER(ctypes.c_int64)
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)


class Sched(ctypes.Structure):
    _fields_ = [("n_warmup", ctypes.c_uint64), ("n_samples", ctypes.c_uint64),
                ("steps_per_sample", ctypes.c_uint64)]


_SIG = [
    ("orc_chacha_block", None, [_u32p, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int, _u32p]),
    ("orc_seed_from_u64", None, [ctypes.c_uint64, _u32p]),
    ("orc_rng_split", None, [ctypes.c_uint64, ctypes.c_size_t, _u64p]),
    ("orc_stream_word", ctypes.c_uint32, [_u32p, ctypes.c_uint64]),
    ("orc_exp", ctypes.c_float, [ctypes.c_float]),
    ("orc_sigmoid", ctypes.c_float, [ctypes.c_float]),
    ("orc_log", ctypes.c_float, [ctypes.c_float]),
    ("orc_gumbel", ctypes.c_float, [ctypes.c_uint32]),
    ("orc_map_f32", None, [ctypes.c_int, _f32p, _f32p, ctypes.c_size_t]),
    ("orc_map_gumbel", None, [_u32p, _f32p, ctypes.c_size_t]),
    ("orc_gumbel_argmax", None,
     [_f32p, _f32p, ctypes.POINTER(ctypes.c_int32), ctypes.c_size_t, ctypes.c_uint32]),
    ("orc_sigmoid_bernoulli", None, [_f32p, _f32p, _f32p, ctypes.c_size_t]),
    ("orc_batch_gather", None,
     [_f32p, ctypes.c_uint64, ctypes.POINTER(ctypes.c_int32), ctypes.c_uint64, ctypes.c_uint32,
      _u32p, ctypes.c_uint32, _f32p]),
    ("orc_lattice_edges", ctypes.c_size_t, [ctypes.c_uint32, ctypes.c_int, _u32p, _u32p]),
    ("orc_lattice_blocks", None, [ctypes.c_uint32, _u32p, _u32p]),
    ("orc_greedy_coloring", ctypes.c_uint32,
     [ctypes.c_uint32, ctypes.c_size_t, _u32p, _u32p, _u32p]),
    ("orc_param_normal", None,
     [ctypes.c_uint64, ctypes.c_size_t, ctypes.c_double, ctypes.c_double, _f32p]),
    ("orc_ising_create", ctypes.c_void_p,
     [ctypes.c_uint32, ctypes.c_size_t, _u32p, _u32p, _f32p, _f32p, ctypes.c_float,
      ctypes.c_uint32, _u32p, _u32p, ctypes.c_uint32, _u32p, _u32p, ctypes.c_char_p,
      ctypes.c_size_t]),
    ("orc_ising_destroy", None, [ctypes.c_void_p]),
    ("orc_ising_set_superblocks", ctypes.c_int,
     [ctypes.c_void_p, ctypes.c_uint32, _u32p, ctypes.c_char_p, ctypes.c_size_t]),
    ("orc_potts_set_superblocks", ctypes.c_int,
     [ctypes.c_void_p, ctypes.c_uint32, _u32p, ctypes.c_char_p, ctypes.c_size_t]),
    ("orc_ising_total", ctypes.c_size_t, [ctypes.c_void_p]),
    ("orc_ising_pos", ctypes.c_int64, [ctypes.c_void_p, ctypes.c_uint32]),
    ("orc_hinton_init", None, [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, _u8p]),
    ("orc_run_blocks", None,
     [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, _u8p, ctypes.c_uint64, ctypes.c_int,
      _u64p]),
    ("orc_estimate_moments", None,
     [ctypes.c_void_p, ctypes.c_uint64, Sched, ctypes.c_uint32, _u8p, _u32p, ctypes.c_size_t,
      _u32p, ctypes.c_size_t, _i64p, _i64p, ctypes.c_int, _u64p]),
    ("orc_sample_states", None,
     [ctypes.c_void_p, ctypes.c_uint64, Sched, ctypes.c_uint32, _u8p, _u8p, ctypes.c_int]),
    ("orc_run_blocks_subset", None,
     [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, _u32p, ctypes.c_uint32, _u8p,
      ctypes.c_uint64, ctypes.c_int]),
    ("orc_ising_gamma", None, [ctypes.c_void_p, _u8p, _f32p]),
    ("orc_ising_energy", None, [ctypes.c_void_p, ctypes.c_uint32, _u8p, _f64p]),
    ("orc_run_blocks_opbyop", None,
     [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, _u8p, ctypes.c_uint64]),
    ("orc_potts_create", ctypes.c_void_p,
     [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_size_t, _u32p, _u32p, _f32p, _f32p,
      ctypes.c_uint32, _u32p, _u32p, ctypes.c_uint32, _u32p, _u32p, ctypes.c_char_p,
      ctypes.c_size_t]),
    ("orc_potts_sample_states", None,
     [ctypes.c_void_p, ctypes.c_uint64, Sched, ctypes.c_uint32, _u16p, _u16p, ctypes.c_int]),
    ("orc_potts_destroy", None, [ctypes.c_void_p]),
    ("orc_potts_total", ctypes.c_size_t, [ctypes.c_void_p]),
    ("orc_potts_run_blocks", None,
     [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, _u16p, ctypes.c_uint64, ctypes.c_int,
      _u64p]),
    ("orc_potts_theta", None, [ctypes.c_void_p, _u16p, _f32p]),
    ("orc_potts_pos", ctypes.c_int64, [ctypes.c_void_p, ctypes.c_uint32]),
    ("orc_potts_energy", None, [ctypes.c_void_p, ctypes.c_uint32, _u16p, _f64p]),
    ("orc_discrete_create", ctypes.c_void_p,
     [ctypes.c_uint32, _u8p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p, ctypes.c_uint32,
      _u32p, _u32p, ctypes.c_uint32, _u32p, _u32p, ctypes.c_char_p, ctypes.c_size_t]),
    ("orc_discrete_destroy", None, [ctypes.c_void_p]),
    ("orc_discrete_set_superblocks", ctypes.c_int,
     [ctypes.c_void_p, ctypes.c_uint32, _u32p, ctypes.c_char_p, ctypes.c_size_t]),
    ("orc_discrete_total", ctypes.c_size_t, [ctypes.c_void_p]),
    ("orc_discrete_pos", ctypes.c_int64, [ctypes.c_void_p, ctypes.c_uint32]),
    ("orc_discrete_params", None, [ctypes.c_void_p, _u16p, _f32p]),
    ("orc_discrete_run_blocks", None,
     [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, _u16p, ctypes.c_uint64, ctypes.c_int,
      _u64p]),
    ("orc_discrete_sample_states", None,
     [ctypes.c_void_p, ctypes.c_uint64, Sched, ctypes.c_uint32, _u16p, _u16p, ctypes.c_int]),
    ("orc_discrete_energy", None, [ctypes.c_void_p, ctypes.c_uint32, _u16p, _f64p]),
    ("orc_rbm_half_sweep", None,
     [ctypes.c_uint32, ctypes.c_uint32, _f32p, _f32p, _f32p, ctypes.c_float, ctypes.c_uint32,
      _u32p, ctypes.c_int, _u8p, _u8p, _u8p, ctypes.c_double, ctypes.c_int]),
]

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        for name, res, args in _SIG:
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _p(a, t):
    return None if a is None else a.ctypes.data_as(ctypes.POINTER(t))


def threads():
    return max(1, min(16, os.cpu_count() or 1))


# ---- rng -----------------------------------------------------------------
def chacha_block(key8, counter, stream=0, rounds=8):
    k = np.ascontiguousarray(np.asarray(key8, np.uint32))
    o = np.zeros(16, np.uint32)
    lib().orc_chacha_block(_p(k, ctypes.c_uint32), counter, stream, rounds, _p(o, ctypes.c_uint32))
    return o


def seed_from_u64(s):
    k = np.zeros(8, np.uint32)
    lib().orc_seed_from_u64(int(s) & (2**64 - 1), _p(k, ctypes.c_uint32))
    return k


def rng_split(key, n):
    o = np.zeros(max(n, 1), np.uint64)
    lib().orc_rng_split(int(key) & (2**64 - 1), n, _p(o, ctypes.c_uint64))
    return [int(x) for x in o[:n]]


def stream_word(key8, w):
    k = np.ascontiguousarray(np.asarray(key8, np.uint32))
    return int(lib().orc_stream_word(_p(k, ctypes.c_uint32), w))


# ---- math ----------------------------------------------------------------
def exp(x):
    return np.float32(lib().orc_exp(float(x)))


def sigmoid(x):
    return np.float32(lib().orc_sigmoid(float(x)))


def log(x):
    return np.float32(lib().orc_log(float(x)))


def gumbel(w):
    return np.float32(lib().orc_gumbel(int(w)))


_MAP_FN = {"exp": 0, "sigmoid": 1, "log": 2, "exp_full": 3, "sigmoid_full": 4, "log_full": 5}


def map_f32(fn, x):
    """Vectorised exp, sigmoid or log ('exp', 'sigmoid', 'log'), or their
    full-range forms ('exp_full', 'sigmoid_full', 'log_full')."""
    x = np.ascontiguousarray(np.asarray(x, np.float32))
    y = np.zeros_like(x)
    lib().orc_map_f32(_MAP_FN[fn], _p(x, ctypes.c_float), _p(y, ctypes.c_float), x.size)
    return y


def gumbel_argmax(logits, u):
    """The reference's kernel-level Gumbel-argmax over rows of [n, q]."""
    logits = np.ascontiguousarray(np.asarray(logits, np.float32))
    u = np.ascontiguousarray(np.asarray(u, np.float32))
    n, q = logits.shape
    out = np.zeros(n, np.int32)
    lib().orc_gumbel_argmax(_p(logits, ctypes.c_float), _p(u, ctypes.c_float),
                            _p(out, ctypes.c_int32), n, q)
    return out


def sigmoid_bernoulli(gamma, u):
    """The reference's kernel-level sigmoid-Bernoulli: (u < sigmoid(2 gamma)) as f32."""
    gamma = np.ascontiguousarray(np.asarray(gamma, np.float32))
    u = np.ascontiguousarray(np.asarray(u, np.float32))
    out = np.zeros_like(gamma)
    lib().orc_sigmoid_bernoulli(_p(gamma, ctypes.c_float), _p(u, ctypes.c_float),
                                _p(out, ctypes.c_float), gamma.size)
    return out


def batch_gather(weights, indices, strides, batch_stride):
    """The reference's batch_gather_fused on flat weights and [batch, n]
    int32 indices (out-of-range linear indices give 0.0)."""
    w = np.ascontiguousarray(np.asarray(weights, np.float32).reshape(-1))
    idx = np.ascontiguousarray(np.asarray(indices, np.int32))
    idx = idx.reshape(idx.shape[0], -1) if idx.ndim else idx.reshape(1, 1)
    st = np.ascontiguousarray(np.asarray(strides, np.uint32).reshape(-1))
    out = np.zeros(idx.shape[0], np.float32)
    lib().orc_batch_gather(_p(w, ctypes.c_float), w.size, _p(idx, ctypes.c_int32), idx.shape[0],
                           idx.shape[1], _p(st, ctypes.c_uint32), int(batch_stride),
                           _p(out, ctypes.c_float))
    return out


def map_gumbel(w):
    w = np.ascontiguousarray(np.asarray(w, np.uint32))
    y = np.zeros(w.shape, np.float32)
    lib().orc_map_gumbel(_p(w, ctypes.c_uint32), _p(y, ctypes.c_float), w.size)
    return y


# ---- graphs --------------------------------------------------------------
def lattice_edges(side, torus=True):
    n = lib().orc_lattice_edges(side, 1 if torus else 0, None, None)
    u = np.zeros(max(n, 1), np.uint32)
    v = np.zeros(max(n, 1), np.uint32)
    lib().orc_lattice_edges(side, 1 if torus else 0, _p(u, ctypes.c_uint32), _p(v, ctypes.c_uint32))
    return np.stack([u[:n], v[:n]], axis=1)


def lattice_blocks(side):
    L = (side + 1) // 2 * 2
    up = np.zeros(L * L // 2, np.uint32)
    lo = np.zeros(L * L // 2, np.uint32)
    lib().orc_lattice_blocks(side, _p(up, ctypes.c_uint32), _p(lo, ctypes.c_uint32))
    return up, lo


def greedy_coloring(n, edges):
    edges = np.ascontiguousarray(np.asarray(edges, np.uint32).reshape(-1, 2))
    u = np.ascontiguousarray(edges[:, 0])
    v = np.ascontiguousarray(edges[:, 1])
    c = np.zeros(max(n, 1), np.uint32)
    k = lib().orc_greedy_coloring(n, u.size, _p(u, ctypes.c_uint32), _p(v, ctypes.c_uint32),
                                  _p(c, ctypes.c_uint32))
    return c[:n], int(k)


def param_normal(seed, n, mean, std):
    o = np.zeros(max(n, 1), np.float32)
    lib().orc_param_normal(seed, n, mean, std, _p(o, ctypes.c_float))
    return o[:n]


def _flat(blocks):
    blocks = [np.asarray(b, np.uint32).reshape(-1) for b in blocks]
    off = np.zeros(len(blocks) + 1, np.uint32)
    for i, b in enumerate(blocks):
        off[i + 1] = off[i] + b.size
    flat = np.ascontiguousarray(np.concatenate(blocks) if blocks else np.zeros(1, np.uint32))
    return off, flat


def _set_superblocks(fn, h, superblocks):
    """superblocks: offsets [n_sb + 1] over the free blocks, or None."""
    if superblocks is None:
        return None
    off = np.ascontiguousarray(np.asarray(superblocks, np.uint32).reshape(-1))
    err = ctypes.create_string_buffer(256)
    if fn(h, max(off.size - 1, 0), _p(off, ctypes.c_uint32), err, 256) != 0:
        raise ValueError(err.value.decode())
    return off


class Ising:
    """Oracle Ising program over free (+ clamped) blocks of node ids;
    superblocks = offsets over the free blocks (None: one per block)."""

    def __init__(self, n_nodes, edges, biases, weights, beta, free_blocks, clamped_blocks=(),
                 superblocks=None):
        edges = np.asarray(edges, np.uint32).reshape(-1, 2)
        self._eu = np.ascontiguousarray(edges[:, 0])
        self._ev = np.ascontiguousarray(edges[:, 1])
        self._b = np.ascontiguousarray(np.asarray(biases, np.float32))
        self._w = np.ascontiguousarray(np.asarray(weights, np.float32))
        foff, fnodes = _flat(free_blocks)
        coff, cnodes = _flat(clamped_blocks)
        self._keep = (foff, fnodes, coff, cnodes)
        err = ctypes.create_string_buffer(256)
        h = lib().orc_ising_create(
            n_nodes, self._eu.size, _p(self._eu, ctypes.c_uint32), _p(self._ev, ctypes.c_uint32),
            _p(self._b, ctypes.c_float), _p(self._w, ctypes.c_float), float(beta),
            len(free_blocks), _p(foff, ctypes.c_uint32), _p(fnodes, ctypes.c_uint32),
            len(clamped_blocks), _p(coff, ctypes.c_uint32), _p(cnodes, ctypes.c_uint32), err, 256)
        if not h:
            raise ValueError(err.value.decode())
        self._h = h
        _set_superblocks(lib().orc_ising_set_superblocks, h, superblocks)
        self.n_total = int(lib().orc_ising_total(h))
        self.free_blocks = [np.asarray(b, np.uint32) for b in free_blocks]
        self.clamped_blocks = [np.asarray(b, np.uint32) for b in clamped_blocks]

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_ising_destroy(self._h)
            self._h = None

    def pos(self, node):
        return int(lib().orc_ising_pos(self._h, int(node)))

    def hinton_init(self, key, C):
        st = np.zeros((C, self.n_total), np.uint8)
        lib().orc_hinton_init(self._h, int(key), C, _p(st, ctypes.c_uint8))
        return st

    def run_blocks(self, key, state, n_iters, n_threads=None):
        st = np.ascontiguousarray(state.copy())
        near = ctypes.c_uint64()
        lib().orc_run_blocks(self._h, int(key), st.shape[0], _p(st, ctypes.c_uint8), n_iters,
                             n_threads or threads(), ctypes.byref(near))
        return st, int(near.value)

    def run_blocks_subset(self, key, C_total, chains, state, n_iters, n_threads=None):
        st = np.ascontiguousarray(state.copy())
        ch = np.ascontiguousarray(np.asarray(chains, np.uint32))
        lib().orc_run_blocks_subset(self._h, int(key), C_total, _p(ch, ctypes.c_uint32), ch.size,
                                    _p(st, ctypes.c_uint8), n_iters, n_threads or threads())
        return st

    def gamma(self, state_row):
        st = np.ascontiguousarray(np.asarray(state_row, np.uint8))
        nf = sum(b.size for b in self.free_blocks)
        out = np.zeros(nf, np.float32)
        lib().orc_ising_gamma(self._h, _p(st, ctypes.c_uint8), _p(out, ctypes.c_float))
        return out

    def run_blocks_opbyop(self, key, state, n_iters):
        st = np.ascontiguousarray(state.copy())
        lib().orc_run_blocks_opbyop(self._h, int(key), st.shape[0], _p(st, ctypes.c_uint8), n_iters)
        return st

    def estimate_moments(self, key, sched, state, nodes, pairs, n_threads=None):
        st = np.ascontiguousarray(state.copy())
        nodes = np.ascontiguousarray(np.asarray(nodes, np.uint32).reshape(-1))
        pairs = np.ascontiguousarray(np.asarray(pairs, np.uint32).reshape(-1, 2))
        ns = np.zeros(max(nodes.size, 1), np.int64)
        es = np.zeros(max(pairs.shape[0], 1), np.int64)
        near = ctypes.c_uint64()
        lib().orc_estimate_moments(self._h, int(key), Sched(*sched), st.shape[0],
                                   _p(st, ctypes.c_uint8), _p(nodes, ctypes.c_uint32), nodes.size,
                                   _p(pairs, ctypes.c_uint32), pairs.shape[0],
                                   _p(ns, ctypes.c_int64), _p(es, ctypes.c_int64),
                                   n_threads or threads(), ctypes.byref(near))
        return ns[:nodes.size], es[:pairs.shape[0]], st, int(near.value)

    def sample_states(self, key, sched, state, n_threads=None):
        st = np.ascontiguousarray(state.copy())
        n_obs = max(int(sched[1]), 1)
        out = np.zeros((n_obs,) + st.shape, np.uint8)
        lib().orc_sample_states(self._h, int(key), Sched(*sched), st.shape[0],
                                _p(st, ctypes.c_uint8), _p(out, ctypes.c_uint8),
                                n_threads or threads())
        return out

    def energy(self, state):
        st = np.ascontiguousarray(state)
        out = np.zeros(st.shape[0], np.float64)
        lib().orc_ising_energy(self._h, st.shape[0], _p(st, ctypes.c_uint8), _p(out, ctypes.c_double))
        return out


class Potts:
    """Oracle categorical program over free (+ clamped) blocks of node ids;
    superblocks as for Ising."""

    def __init__(self, n_nodes, q, edges, W, bias, free_blocks, clamped_blocks=(),
                 superblocks=None):
        edges = np.asarray(edges, np.uint32).reshape(-1, 2)
        self._eu = np.ascontiguousarray(edges[:, 0])
        self._ev = np.ascontiguousarray(edges[:, 1])
        self._W = np.ascontiguousarray(np.asarray(W, np.float32).reshape(-1))
        self._b = np.ascontiguousarray(np.asarray(bias, np.float32).reshape(-1))
        foff, fnodes = _flat(free_blocks)
        coff, cnodes = _flat(clamped_blocks)
        self._keep = (foff, fnodes, coff, cnodes)
        err = ctypes.create_string_buffer(256)
        h = lib().orc_potts_create(n_nodes, q, self._eu.size, _p(self._eu, ctypes.c_uint32),
                                   _p(self._ev, ctypes.c_uint32), _p(self._W, ctypes.c_float),
                                   _p(self._b, ctypes.c_float), len(free_blocks),
                                   _p(foff, ctypes.c_uint32), _p(fnodes, ctypes.c_uint32),
                                   len(clamped_blocks), _p(coff, ctypes.c_uint32),
                                   _p(cnodes, ctypes.c_uint32), err, 256)
        if not h:
            raise ValueError(err.value.decode())
        self._h = h
        _set_superblocks(lib().orc_potts_set_superblocks, h, superblocks)
        self.q = int(q)
        self.n_total = int(lib().orc_potts_total(h))

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_potts_destroy(self._h)
            self._h = None

    # states cross the C interface as uint16 [C][n_total]; results come back as
    # uint8 when every category fits a byte (q <= 256), else uint16
    def _u16(self, state):
        st = np.asarray(state)
        if st.size and (st.min() < 0 or st.max() >= self.q):
            raise ValueError("category out of range")
        return np.ascontiguousarray(st.astype(np.uint16))

    def _out(self, st):
        return st.astype(np.uint8) if self.q <= 256 else st

    def theta(self, state_row):
        st = self._u16(state_row)
        out = np.zeros((self.n_total, self.q), np.float32)
        lib().orc_potts_theta(self._h, _p(st, ctypes.c_uint16), _p(out, ctypes.c_float))
        return out

    def pos(self, node):
        return int(lib().orc_potts_pos(self._h, int(node)))

    def energy(self, state):
        st = self._u16(np.asarray(state).reshape(-1, self.n_total))
        out = np.zeros(st.shape[0], np.float64)
        lib().orc_potts_energy(self._h, st.shape[0], _p(st, ctypes.c_uint16), _p(out, ctypes.c_double))
        return out

    def sample_states(self, key, sched, state, n_threads=None):
        st = self._u16(state)
        n_obs = max(int(sched[1]), 1)
        out = np.zeros((n_obs,) + st.shape, np.uint16)
        lib().orc_potts_sample_states(self._h, int(key), Sched(*sched), st.shape[0],
                                      _p(st, ctypes.c_uint16), _p(out, ctypes.c_uint16),
                                      n_threads or threads())
        return self._out(out)

    def run_blocks(self, key, state, n_iters, n_threads=None):
        st = self._u16(state)
        near = ctypes.c_uint64()
        lib().orc_potts_run_blocks(self._h, int(key), st.shape[0], _p(st, ctypes.c_uint16), n_iters,
                                   n_threads or threads(), ctypes.byref(near))
        return self._out(st), int(near.value)


class _Factor(ctypes.Structure):
    _fields_ = [("n_spin", ctypes.c_uint32), ("n_cat", ctypes.c_uint32), ("batch", ctypes.c_uint32),
                ("d1", ctypes.c_uint32), ("d2", ctypes.c_uint32), ("nodes", _u32p), ("w", _f32p),
                ("square", ctypes.c_uint32)]


class Discrete:
    """Oracle program over general discrete factors.  kinds[n] = 0 spin, 1
    categorical (q categories); factors = [(spin_groups, cat_groups, W)] or
    [(spin_groups, cat_groups, W, square)] with W of shape [batch, d1, d2];
    superblocks as for Ising."""

    def __init__(self, n_nodes, kinds, q, factors, free_blocks, clamped_blocks=(),
                 superblocks=None):
        self._kinds = np.ascontiguousarray(np.asarray(kinds, np.uint8).reshape(-1))
        keep = []
        arr = (_Factor * max(len(factors), 1))()
        for i, f in enumerate(factors):
            sg, cg, W = f[:3]
            square = int(bool(f[3])) if len(f) > 3 else 0
            groups = [np.asarray(g, np.uint32).reshape(-1) for g in list(sg) + list(cg)]
            batch = groups[0].size if groups else 0
            nodes = np.ascontiguousarray(np.concatenate(groups) if groups else np.zeros(1, np.uint32))
            W = np.ascontiguousarray(np.asarray(W, np.float32))
            W = W.reshape(W.shape[0], *(list(W.shape[1:]) + [1, 1])[:2])
            keep += [nodes, W]
            arr[i] = _Factor(len(sg), len(cg), batch, W.shape[1], W.shape[2],
                             _p(nodes, ctypes.c_uint32), _p(W, ctypes.c_float), square)
        foff, fnodes = _flat(free_blocks)
        coff, cnodes = _flat(clamped_blocks)
        self._keep = (keep, arr, foff, fnodes, coff, cnodes)
        err = ctypes.create_string_buffer(256)
        h = lib().orc_discrete_create(n_nodes, _p(self._kinds, ctypes.c_uint8), int(q), len(factors),
                                      ctypes.cast(arr, ctypes.c_void_p), len(free_blocks),
                                      _p(foff, ctypes.c_uint32), _p(fnodes, ctypes.c_uint32),
                                      len(clamped_blocks), _p(coff, ctypes.c_uint32),
                                      _p(cnodes, ctypes.c_uint32), err, 256)
        if not h:
            raise ValueError(err.value.decode())
        self._h = h
        _set_superblocks(lib().orc_discrete_set_superblocks, h, superblocks)
        self.q = int(q)
        self.n_total = int(lib().orc_discrete_total(h))
        self.free_blocks = [np.asarray(b, np.uint32) for b in free_blocks]

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_discrete_destroy(self._h)
            self._h = None

    def pos(self, node):
        return int(lib().orc_discrete_pos(self._h, int(node)))

    # states cross the C interface as uint16 [C][n_total]; results come back as
    # uint8 when every category fits a byte (q <= 256), else uint16
    def _u16(self, state):
        st = np.asarray(state)
        if st.size and (st.min() < 0 or st.max() >= max(self.q, 2)):
            raise ValueError("state value out of range")
        return np.ascontiguousarray(st.astype(np.uint16))

    def _out(self, st):
        return st.astype(np.uint8) if self.q <= 256 else st

    def params(self, state_row):
        """[n_free_total, max(q, 1)]: gamma in column 0 for spin positions,
        theta for categorical ones."""
        st = self._u16(state_row)
        nf = sum(b.size for b in self.free_blocks)
        out = np.zeros((nf, max(self.q, 1)), np.float32)
        lib().orc_discrete_params(self._h, _p(st, ctypes.c_uint16), _p(out, ctypes.c_float))
        return out

    def run_blocks(self, key, state, n_iters, n_threads=None):
        st = self._u16(state).copy()
        near = ctypes.c_uint64()
        lib().orc_discrete_run_blocks(self._h, int(key), st.shape[0], _p(st, ctypes.c_uint16),
                                      n_iters, n_threads or threads(), ctypes.byref(near))
        return self._out(st), int(near.value)

    def sample_states(self, key, sched, state, n_threads=None):
        st = self._u16(state).copy()
        n_obs = max(int(sched[1]), 1)
        out = np.zeros((n_obs,) + st.shape, np.uint16)
        lib().orc_discrete_sample_states(self._h, int(key), Sched(*sched), st.shape[0],
                                         _p(st, ctypes.c_uint16), _p(out, ctypes.c_uint16),
                                         n_threads or threads())
        return self._out(out)

    def energy(self, state):
        st = self._u16(np.asarray(state).reshape(-1, self.n_total))
        out = np.zeros(st.shape[0], np.float64)
        lib().orc_discrete_energy(self._h, st.shape[0], _p(st, ctypes.c_uint16),
                                  _p(out, ctypes.c_double))
        return out


def rbm_half_sweep(W, bv, bh, beta, key8, blk, sv, sh, tol=1e-5, n_threads=None):
    W = np.ascontiguousarray(np.asarray(W, np.float32))
    V, H = W.shape
    bv = np.ascontiguousarray(np.asarray(bv, np.float32))
    bh = np.ascontiguousarray(np.asarray(bh, np.float32))
    key8 = np.ascontiguousarray(np.asarray(key8, np.uint32).reshape(-1))
    sv = np.ascontiguousarray(sv.copy())
    sh = np.ascontiguousarray(sh.copy())
    C = sv.shape[0]
    n = V if blk == 0 else H
    near = np.zeros((C, n), np.uint8)
    lib().orc_rbm_half_sweep(V, H, _p(W, ctypes.c_float), _p(bv, ctypes.c_float),
                             _p(bh, ctypes.c_float), float(beta), C, _p(key8, ctypes.c_uint32), blk,
                             _p(sv, ctypes.c_uint8), _p(sh, ctypes.c_uint8), _p(near, ctypes.c_uint8),
                             tol, n_threads or threads())
    return sv, sh, near
