"""ctypes binding of libthrml_hip.so (the C ABI declared in include/thrml_hip.h).

The library is the product path: there is no Python or CPU fallback.  If the
shared object is missing, every call raises ThrmlError.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.normpath(os.path.join(_HERE, "..", "libthrml_hip.so"))

THRML_OK = 0
THRML_EINVAL = -1
THRML_EHIP = -2
THRML_ENOMEM = -3
THRML_EUNSUPPORTED = -4
DTYPE_U8 = 0
DTYPE_F32 = 1

KIND_NAMES = {0: "lattice", 1: "csr", 2: "potts", 3: "dense", 4: "discrete"}


class ThrmlError(RuntimeError):
    """Error returned by the library (the reference's Err(String))."""

    def __init__(self, code, msg):
        super().__init__(msg)
        self.code = code


c_u32p = ctypes.POINTER(ctypes.c_uint32)
c_u64p = ctypes.POINTER(ctypes.c_uint64)
c_i64p = ctypes.POINTER(ctypes.c_int64)
c_f32p = ctypes.POINTER(ctypes.c_float)
c_f64p = ctypes.POINTER(ctypes.c_double)
c_u16p = ctypes.POINTER(ctypes.c_uint16)
c_u8p = ctypes.POINTER(ctypes.c_uint8)


class IsingDesc(ctypes.Structure):
    _fields_ = [
        ("n_nodes", ctypes.c_uint32),
        ("n_edges", ctypes.c_uint64),
        ("edge_u", c_u32p),
        ("edge_v", c_u32p),
        ("biases", c_f32p),
        ("weights", c_f32p),
        ("beta", ctypes.c_float),
        ("n_free_blocks", ctypes.c_uint32),
        ("free_offsets", c_u32p),
        ("free_nodes", c_u32p),
        ("n_clamped_blocks", ctypes.c_uint32),
        ("clamped_offsets", c_u32p),
        ("clamped_nodes", c_u32p),
        ("flags", ctypes.c_uint32),
        ("n_superblocks", ctypes.c_uint32),
        ("superblock_offsets", c_u32p),
    ]


ISING_DENSE = 2
RBM_CLAMP = {None: 0, "visible": 1, "hidden": 2}


class PottsDesc(ctypes.Structure):
    _fields_ = [
        ("n_nodes", ctypes.c_uint32),
        ("q", ctypes.c_uint32),
        ("n_edges", ctypes.c_uint64),
        ("edge_u", c_u32p),
        ("edge_v", c_u32p),
        ("weights", c_f32p),
        ("biases", c_f32p),
        ("n_free_blocks", ctypes.c_uint32),
        ("free_offsets", c_u32p),
        ("free_nodes", c_u32p),
        ("n_clamped_blocks", ctypes.c_uint32),
        ("clamped_offsets", c_u32p),
        ("clamped_nodes", c_u32p),
        ("n_superblocks", ctypes.c_uint32),
        ("superblock_offsets", c_u32p),
    ]


class RbmDesc(ctypes.Structure):
    _fields_ = [
        ("n_visible", ctypes.c_uint32),
        ("n_hidden", ctypes.c_uint32),
        ("weights_bf16", c_u16p),
        ("bias_visible", c_f32p),
        ("bias_hidden", c_f32p),
        ("beta", ctypes.c_float),
        ("clamped", ctypes.c_uint32),
        ("weights_f32", c_f32p),
    ]


class DiscreteFactor(ctypes.Structure):
    _fields_ = [
        ("n_spin_groups", ctypes.c_uint32),
        ("n_cat_groups", ctypes.c_uint32),
        ("batch", ctypes.c_uint32),
        ("d1", ctypes.c_uint32),
        ("d2", ctypes.c_uint32),
        ("nodes", c_u32p),
        ("weights", c_f32p),
        ("flags", ctypes.c_uint32),
    ]


THRML_FACTOR_SQUARE = 1


class DiscreteDesc(ctypes.Structure):
    _fields_ = [
        ("n_nodes", ctypes.c_uint32),
        ("node_kind", c_u8p),
        ("q", ctypes.c_uint32),
        ("n_factors", ctypes.c_uint32),
        ("factors", ctypes.POINTER(DiscreteFactor)),
        ("n_free_blocks", ctypes.c_uint32),
        ("free_offsets", c_u32p),
        ("free_nodes", c_u32p),
        ("n_clamped_blocks", ctypes.c_uint32),
        ("clamped_offsets", c_u32p),
        ("clamped_nodes", c_u32p),
        ("n_superblocks", ctypes.c_uint32),
        ("superblock_offsets", c_u32p),
    ]


class Schedule(ctypes.Structure):
    _fields_ = [
        ("n_warmup", ctypes.c_uint64),
        ("n_samples", ctypes.c_uint64),
        ("steps_per_sample", ctypes.c_uint64),
    ]


# int observe(void *user, uint64_t iteration, thrml_state *st, void *hip_stream)
OBSERVE_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p,
                              ctypes.c_void_p)


class ProgInfo(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_uint32),
        ("n_free_blocks", ctypes.c_uint32),
        ("n_clamped_blocks", ctypes.c_uint32),
        ("n_total", ctypes.c_uint64),
        ("device_bytes", ctypes.c_uint64),
        ("dense_pieces", ctypes.c_uint32),
    ]


# (name, restype, argtypes); every symbol declared in include/thrml_hip.h
SIGNATURES = [
    ("thrml_version", ctypes.c_int, []),
    ("thrml_last_error", ctypes.c_char_p, []),
    ("thrml_ctx_create", ctypes.c_int, [ctypes.c_int, ctypes.POINTER(ctypes.c_void_p)]),
    ("thrml_ctx_destroy", None, [ctypes.c_void_p]),
    ("thrml_ctx_set_stream", ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
    ("thrml_ctx_get_stream", ctypes.c_void_p, [ctypes.c_void_p]),
    ("thrml_ctx_synchronize", ctypes.c_int, [ctypes.c_void_p]),
    ("thrml_ctx_enable_timing", ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
    ("thrml_ctx_kernel_time", ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, c_f64p, c_u64p]),
    ("thrml_rng_split", ctypes.c_int, [ctypes.c_uint64, ctypes.c_uint64, c_u64p]),
    ("thrml_lattice_edges", ctypes.c_int64, [ctypes.c_uint32, ctypes.c_int, c_u32p, c_u32p]),
    ("thrml_lattice_blocks", ctypes.c_int, [ctypes.c_uint32, c_u32p, c_u32p]),
    ("thrml_greedy_coloring", ctypes.c_int64,
     [ctypes.c_uint32, ctypes.c_uint64, c_u32p, c_u32p, c_u32p]),
    ("thrml_erdos_renyi", ctypes.c_int64,
     [ctypes.c_uint32, ctypes.c_double, ctypes.c_uint64, c_u32p, c_u32p, ctypes.c_uint64]),
    ("thrml_double_grid", ctypes.c_int64,
     [ctypes.c_uint32, c_u32p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint64, c_u32p, c_u32p,
      c_u32p]),
    ("thrml_param_normal", ctypes.c_int,
     [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_double, ctypes.c_double, c_f32p]),
    ("thrml_ising_program_create", ctypes.c_int,
     [ctypes.c_void_p, ctypes.POINTER(IsingDesc), ctypes.POINTER(ctypes.c_void_p)]),
    ("thrml_potts_program_create", ctypes.c_int,
     [ctypes.c_void_p, ctypes.POINTER(PottsDesc), ctypes.POINTER(ctypes.c_void_p)]),
    ("thrml_rbm_program_create", ctypes.c_int,
     [ctypes.c_void_p, ctypes.POINTER(RbmDesc), ctypes.POINTER(ctypes.c_void_p)]),
    ("thrml_discrete_program_create", ctypes.c_int,
     [ctypes.c_void_p, ctypes.POINTER(DiscreteDesc), ctypes.POINTER(ctypes.c_void_p)]),
    ("thrml_prog_destroy", None, [ctypes.c_void_p]),
    ("thrml_prog_get_info", ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ProgInfo)]),
    ("thrml_prog_block", ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, c_u64p, c_u64p]),
    ("thrml_state_create", ctypes.c_int,
     [ctypes.c_void_p, ctypes.c_uint32, ctypes.POINTER(ctypes.c_void_p)]),
    ("thrml_state_destroy", None, [ctypes.c_void_p]),
    ("thrml_state_set_block", ctypes.c_int,
     [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]),
    ("thrml_state_get_block", ctypes.c_int,
     [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]),
    ("thrml_hinton_init", ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p]),
    ("thrml_run_blocks", ctypes.c_int,
     [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64]),
    ("thrml_run_blocks_noalloc", ctypes.c_int,
     [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64]),
    ("thrml_estimate_moments", ctypes.c_int,
     [ctypes.c_void_p, ctypes.c_uint64, Schedule, ctypes.c_void_p, c_u32p, ctypes.c_uint64,
      c_u32p, ctypes.c_uint64, c_i64p, c_i64p]),
    ("thrml_moments_create", ctypes.c_int,
     [ctypes.c_void_p, c_u32p, ctypes.c_uint64, c_u32p, ctypes.c_uint64,
      ctypes.POINTER(ctypes.c_void_p)]),
    ("thrml_moments_destroy", None, [ctypes.c_void_p]),
    ("thrml_moments_run", ctypes.c_int,
     [ctypes.c_void_p, ctypes.c_uint64, Schedule, ctypes.c_void_p, ctypes.c_void_p,
      ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]),
    ("thrml_observer_create", ctypes.c_int,
     [ctypes.c_void_p, c_u64p, ctypes.c_uint64, c_u32p, ctypes.c_int,
      ctypes.POINTER(ctypes.c_void_p)]),
    ("thrml_observer_destroy", None, [ctypes.c_void_p]),
    ("thrml_observer_run", ctypes.c_int,
     [ctypes.c_void_p, ctypes.c_uint64, Schedule, ctypes.c_void_p, ctypes.c_void_p,
      ctypes.c_void_p, ctypes.c_int]),
    ("thrml_sample_with_observer", ctypes.c_int,
     [ctypes.c_void_p, ctypes.c_uint64, Schedule, ctypes.c_void_p, ctypes.c_void_p,
      ctypes.c_void_p]),
    ("thrml_sample_states", ctypes.c_int,
     [ctypes.c_void_p, ctypes.c_uint64, Schedule, ctypes.c_void_p, c_u8p]),
    ("thrml_sample_states_as", ctypes.c_int,
     [ctypes.c_void_p, ctypes.c_uint64, Schedule, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]),
    ("thrml_ising_energy", ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, c_f64p]),
    ("thrml_potts_energy", ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, c_f64p]),
    ("thrml_discrete_energy", ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, c_f64p]),
    ("thrml_rbm_half_sweep", ctypes.c_int,
     [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, c_u32p]),
    ("thrml_sigmoid_bernoulli", ctypes.c_int,
     [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64]),
    ("thrml_gumbel_argmax", ctypes.c_int,
     [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64,
      ctypes.c_uint32]),
    ("thrml_batch_gather", ctypes.c_int,
     [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint64,
      ctypes.c_uint32, c_u32p, ctypes.c_uint32, ctypes.c_void_p]),
    ("thrml_fast_math_check", ctypes.c_int, [ctypes.c_void_p, c_f32p]),
    ("thrml_fast_math_status", ctypes.c_int,
     [ctypes.c_void_p, c_f32p, ctypes.POINTER(ctypes.c_int)]),
    ("thrml_fast_math_bounds_ok", ctypes.c_int, [c_f32p]),
]

_lib = None


def load():
    """Load the shared library (once).  Raises ThrmlError if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ThrmlError(THRML_EINVAL, f"{LIB_PATH} is not built; run __graft_entry__.build()")
    # One HIP runtime per process.  PyTorch-ROCm ships its own libamdhip64 /
    # libhsa-runtime64 and asks for them by a name that does not match an
    # already loaded /opt/rocm copy, so loading this library first would put a
    # second HSA runtime into the process and torch would then find no GPU.
    # Loading torch first lets this library bind to torch's runtime by SONAME.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(LIB_PATH)
    for name, res, args in SIGNATURES:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc):
    if rc < 0:
        msg = load().thrml_last_error()
        raise ThrmlError(rc, msg.decode() if msg else f"error {rc}")
    return rc


def ptr(arr, ctype):
    """ctypes pointer to a contiguous numpy array (None -> NULL)."""
    if arr is None:
        return None
    return arr.ctypes.data_as(ctypes.POINTER(ctype))
