"""Python mirror of thrml-rs's sampling API over libthrml_hip.so.

Names, argument meaning and errors follow the reference crates
(paths relative to the thrml-rs repository root):

  RngKey                      crates/thrml-samplers/src/rng.rs:10-44
  SamplingSchedule            crates/thrml-samplers/src/schedule.rs:4-20
  Block                       crates/thrml-core/src/block.rs:5-45
  IsingEBM                    crates/thrml-models/src/ising.rs:26-149
  IsingSamplingProgram        crates/thrml-models/src/ising.rs:342-388
  CategoricalProgram          crates/thrml-models/src/factor.rs:152-185 with
                              CategoricalGibbsConditional (softmax.rs:228-271)
  RbmProgram                  dense bipartite IsingEBM (no reference type)
  hinton_init                 crates/thrml-models/src/ising.rs:602-673
  run_blocks                  crates/thrml-samplers/src/sampling.rs:81-106
  sample_states               crates/thrml-samplers/src/sampling.rs:128-156
  estimate_moments            crates/thrml-models/src/ising.rs:455-505
  make_nearest_neighbor_lattice  crates/thrml-models/src/graph_utils.rs:177-243
  greedy_coloring, coloring_to_blocks  crates/thrml-examples/src/lib.rs:114-205

Nodes are integers 0..n_nodes-1 (the reference's Node objects carry a global
id; here the id is the node).  States are numpy arrays [n_chains, block_len]
(uint8 or float32 0/1, the reference's representation) or a DeviceState that
keeps the chains resident on the GPU between calls.  Every call goes through
the HIP library; nothing here computes a sweep on the CPU.
"""
import ctypes
import sys
import weakref

import numpy as np

from . import _lib
from ._lib import ThrmlError, check, load, ptr

__all__ = [
    "ThrmlError", "Device", "RngKey", "SamplingSchedule", "Block", "IsingEBM",
    "IsingSamplingProgram", "CategoricalProgram", "RbmProgram", "DeviceState", "hinton_init",
    "DiscreteEBMFactor", "SpinEBMFactor", "CategoricalEBMFactor", "SquareDiscreteEBMFactor",
    "SquareCategoricalEBMFactor", "FactorSamplingProgram",
    "discrete_energy",
    "run_blocks", "sample_states", "sample_with_observation", "AbstractObserver",
    "estimate_moments", "ising_moment_spec",
    "IsingTrainingSpec", "estimate_kl_grad", "ising_energy", "potts_energy", "energy",
    "MomentAccumulatorObserver", "make_nearest_neighbor_lattice",
    "greedy_coloring", "coloring_to_blocks", "erdos_renyi", "double_grid", "param_normal", "bf16_round",
]


# ---------------------------------------------------------------------------
class Device:
    """A HIP device and stream (the reference's WgpuDevice, backend.rs:55-71)."""

    def __init__(self, ordinal=0):
        lib = load()
        h = ctypes.c_void_p()
        check(lib.thrml_ctx_create(int(ordinal), ctypes.byref(h)))
        self._h = h
        self.ordinal = ordinal
        # live objects made on this context, closed before it (the C ABI
        # destroys contexts last)
        self._programs = weakref.WeakSet()
        self._dependents = weakref.WeakSet()

    @property
    def handle(self):
        return self._h

    def synchronize(self):
        check(load().thrml_ctx_synchronize(self._h))

    def set_stream(self, hip_stream):
        check(load().thrml_ctx_set_stream(self._h, ctypes.c_void_p(hip_stream)))

    @property
    def stream(self):
        return load().thrml_ctx_get_stream(self._h)

    def fast_math_check(self):
        """(max Gumbel score error, max relative error of the hardware e^-x,
        max relative error of the exact sigmoid) of the kernels' hardware-math
        fast paths (thrml_fast_math_check)."""
        out = (ctypes.c_float * 3)()
        check(load().thrml_fast_math_check(self._h, out))
        return float(out[0]), float(out[1]), float(out[2])

    def fast_math_status(self):
        """((gumbel, exp, sigmoid) errors, ok) of the self-check the library
        ran at this device's first program creation and keeps
        (thrml_fast_math_status)."""
        out = (ctypes.c_float * 3)()
        ok = ctypes.c_int()
        check(load().thrml_fast_math_status(self._h, out, ctypes.byref(ok)))
        return (float(out[0]), float(out[1]), float(out[2])), bool(ok.value)

    def enable_timing(self, on=True, span=False):
        """HIP-event timing of the library's launches: an event pair around
        each launch, or with span=True one span over all of them."""
        check(load().thrml_ctx_enable_timing(self._h, (2 if span else 1) if on else 0))

    def kernel_time(self, kernel=0):
        """(average milliseconds, launches) of the sweep (0) or moment (1) kernel."""
        ms = ctypes.c_double()
        n = ctypes.c_uint64()
        check(load().thrml_ctx_kernel_time(self._h, kernel, ctypes.byref(ms), ctypes.byref(n)))
        return ms.value, n.value

    def close(self):
        """Destroys the context, after closing the states, moment observers
        and programs still open on it."""
        if getattr(self, "_h", None) is not None and self._h.value:
            for o in list(getattr(self, "_dependents", ())):
                o.close()
            for p in list(getattr(self, "_programs", ())):
                p.close()
            load().thrml_ctx_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        # at interpreter exit the HIP runtime may already be gone: leak instead
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:
            pass


def _register(device, obj, program=False):
    (device._programs if program else device._dependents).add(obj)


# ---------------------------------------------------------------------------
class RngKey:
    """JAX-style key; split = ChaCha8Rng::seed_from_u64 + next_u64 (rng.rs:20-38)."""

    __slots__ = ("seed",)

    def __init__(self, seed):
        self.seed = int(seed) & 0xFFFFFFFFFFFFFFFF

    def split(self, n):
        n = int(n)
        if n == 0:
            return []
        out = np.zeros(n, dtype=np.uint64)
        check(load().thrml_rng_split(self.seed, n, ptr(out, ctypes.c_uint64)))
        return [RngKey(int(x)) for x in out]

    def split_two(self):
        a, b = self.split(2)
        return a, b

    def __eq__(self, other):
        return isinstance(other, RngKey) and other.seed == self.seed

    def __hash__(self):
        return hash(self.seed)

    def __repr__(self):
        return f"RngKey({self.seed})"


class SamplingSchedule:
    def __init__(self, n_warmup, n_samples, steps_per_sample):
        self.n_warmup = int(n_warmup)
        self.n_samples = int(n_samples)
        self.steps_per_sample = int(steps_per_sample)

    def _c(self):
        return _lib.Schedule(self.n_warmup, self.n_samples, self.steps_per_sample)


class Block:
    """A non-empty list of node ids (block.rs:11-27)."""

    def __init__(self, nodes):
        nodes = np.ascontiguousarray(np.asarray(nodes, dtype=np.uint32).reshape(-1))
        if nodes.size == 0:
            raise ThrmlError(_lib.THRML_EINVAL, "Block cannot be empty")
        self.nodes = nodes

    def __len__(self):
        return int(self.nodes.size)


def _is_superblock(item):
    # a list of blocks, or an empty list (an empty superblock samples nothing;
    # a block cannot be empty)
    if isinstance(item, Block) or not isinstance(item, (list, tuple)):
        return False
    return all(isinstance(x, (Block, list, tuple, np.ndarray)) for x in item)


def _super_blocks(free_super_blocks):
    """BlockGibbsSpec::new's flattening (program.rs:28-64): each item is a
    block or a superblock (a list of blocks).  Returns the free blocks in
    order, the sampling order (block indices per superblock) and the
    superblock offsets (None when every superblock holds one block)."""
    blocks, order = [], []
    for item in free_super_blocks:
        group = list(item) if _is_superblock(item) else [item]
        order.append(list(range(len(blocks), len(blocks) + len(group))))
        blocks.extend(group)
    if all(len(g) == 1 for g in order):
        return blocks, order, None
    off = np.zeros(len(order) + 1, dtype=np.uint32)
    for i, g in enumerate(order):
        off[i + 1] = off[i] + len(g)
    return blocks, order, off


def _blocks_flat(blocks):
    blocks = [b if isinstance(b, Block) else Block(b) for b in blocks]
    off = np.zeros(len(blocks) + 1, dtype=np.uint32)
    for i, b in enumerate(blocks):
        off[i + 1] = off[i] + len(b)
    flat = (np.concatenate([b.nodes for b in blocks]).astype(np.uint32) if blocks
            else np.zeros(1, np.uint32))
    return blocks, off, np.ascontiguousarray(flat)


# ---------------------------------------------------------------------------
class IsingEBM:
    """E(s) = -beta (sum_i b_i s_i + sum_(i,j) J_ij s_i s_j) (ising.rs:22-149)."""

    def __init__(self, n_nodes, edges, biases, weights, beta=1.0):
        self.n_nodes = int(n_nodes)
        edges = np.asarray(edges, dtype=np.uint32).reshape(-1, 2)
        self.edge_u = np.ascontiguousarray(edges[:, 0])
        self.edge_v = np.ascontiguousarray(edges[:, 1])
        self.biases = np.ascontiguousarray(np.asarray(biases, dtype=np.float32).reshape(-1))
        self.weights = np.ascontiguousarray(np.asarray(weights, dtype=np.float32).reshape(-1))
        self.beta = float(np.float32(beta))
        if self.biases.size != self.n_nodes:
            raise ThrmlError(_lib.THRML_EINVAL, "biases must have one entry per node")
        if self.weights.size != self.edge_u.size:
            raise ThrmlError(_lib.THRML_EINVAL, "weights must have one entry per edge")

    @property
    def edges(self):
        return np.stack([self.edge_u, self.edge_v], axis=1)


class _Program:
    _h = None

    def _info(self):
        info = _lib.ProgInfo()
        check(load().thrml_prog_get_info(self._h, ctypes.byref(info)))
        return info

    @property
    def kind(self):
        return _lib.KIND_NAMES[self._info().kind]

    @property
    def n_total(self):
        return int(self._info().n_total)

    @property
    def device_bytes(self):
        return int(self._info().device_bytes)

    @property
    def dense_pieces(self):
        """bf16 pieces per weight of a dense program (1..3), 0 for other kinds."""
        return int(self._info().dense_pieces)

    def block_range(self, b):
        off = ctypes.c_uint64()
        n = ctypes.c_uint64()
        check(load().thrml_prog_block(self._h, int(b), ctypes.byref(off), ctypes.byref(n)))
        return int(off.value), int(n.value)

    def new_state(self, n_chains):
        return DeviceState(self, n_chains)

    def close(self):
        if self._h is not None and self._h.value:
            load().thrml_prog_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        # at interpreter exit the HIP runtime may already be gone: leak instead
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:
            pass


class IsingSamplingProgram(_Program):
    """IsingSamplingProgram::new(ebm, free_blocks, clamped_blocks, device).

    Every model runs on a kernel that sums in the reference's slot order
    (kind "lattice" or "csr"), bit for bit, unless dense=True: then a model
    whose edges are exactly the complete bipartite graph between its two
    blocks (at least 64 nodes each side; an RBM) runs on the matrix-core
    kernel (kind "dense"), with f32 weights held exactly as up to three bf16
    pieces.  Its f32 summation order differs from the slot order, so its
    decisions may differ from the reference's where |2 gamma - logit u| <
    1e-5 (threshold sites).

    An entry of free_blocks may be a superblock (a list of blocks), as
    BlockGibbsSpec::new takes them (program.rs:28-64): its blocks are sampled
    from the state before it and written after it (sampling.rs:39-60)."""

    def __init__(self, ebm, free_blocks, clamped_blocks, device, dense=False):
        self.device = device
        self.ebm = ebm
        flat, self.sampling_order, sboff = _super_blocks(free_blocks)
        fb, foff, fnodes = _blocks_flat(flat)
        cb, coff, cnodes = _blocks_flat(clamped_blocks)
        self.free_blocks, self.clamped_blocks = fb, cb
        self._keep = (foff, fnodes, coff, cnodes, sboff)
        d = _lib.IsingDesc(
            ebm.n_nodes, ebm.edge_u.size, ptr(ebm.edge_u, ctypes.c_uint32),
            ptr(ebm.edge_v, ctypes.c_uint32), ptr(ebm.biases, ctypes.c_float),
            ptr(ebm.weights, ctypes.c_float), ebm.beta, len(fb), ptr(foff, ctypes.c_uint32),
            ptr(fnodes, ctypes.c_uint32), len(cb), ptr(coff, ctypes.c_uint32) if cb else None,
            ptr(cnodes, ctypes.c_uint32) if cb else None, _lib.ISING_DENSE if dense else 0,
            0 if sboff is None else sboff.size - 1, ptr(sboff, ctypes.c_uint32))
        h = ctypes.c_void_p()
        check(load().thrml_ising_program_create(device.handle, ctypes.byref(d), ctypes.byref(h)))
        self._h = h
        _register(device, self, program=True)


class CategoricalProgram(_Program):
    """Potts model: bias factor + CategoricalEBMFactor([U, V], W[E, q, q]),
    CategoricalGibbsConditional(q, 0) per free block; the global state is the
    free blocks then the clamped blocks (factor.rs:152-185).  free_blocks
    may hold superblocks, as for IsingSamplingProgram.  q is 2..65536 (one
    byte of state per node up to 256 categories, two above; such states
    read back as uint16)."""

    def __init__(self, n_nodes, q, edges, weights, biases, free_blocks, device,
                 clamped_blocks=()):
        self.device = device
        self.q = int(q)
        edges = np.asarray(edges, dtype=np.uint32).reshape(-1, 2)
        eu = np.ascontiguousarray(edges[:, 0])
        ev = np.ascontiguousarray(edges[:, 1])
        W = np.ascontiguousarray(np.asarray(weights, dtype=np.float32).reshape(-1))
        bias = np.ascontiguousarray(np.asarray(biases, dtype=np.float32).reshape(-1))
        flat, self.sampling_order, sboff = _super_blocks(free_blocks)
        fb, foff, fnodes = _blocks_flat(flat)
        cb, coff, cnodes = _blocks_flat(clamped_blocks)
        self.free_blocks, self.clamped_blocks = fb, cb
        self._keep = (eu, ev, W, bias, foff, fnodes, coff, cnodes, sboff)
        d = _lib.PottsDesc(int(n_nodes), self.q, eu.size, ptr(eu, ctypes.c_uint32),
                           ptr(ev, ctypes.c_uint32), ptr(W, ctypes.c_float),
                           ptr(bias, ctypes.c_float), len(fb), ptr(foff, ctypes.c_uint32),
                           ptr(fnodes, ctypes.c_uint32), len(cb),
                           ptr(coff, ctypes.c_uint32) if cb else None,
                           ptr(cnodes, ctypes.c_uint32) if cb else None,
                           0 if sboff is None else sboff.size - 1, ptr(sboff, ctypes.c_uint32))
        h = ctypes.c_void_p()
        check(load().thrml_potts_program_create(device.handle, ctypes.byref(d), ctypes.byref(h)))
        self._h = h
        _register(device, self, program=True)


class DiscreteEBMFactor:
    """DiscreteEBMFactor::new(spin_node_groups, categorical_node_groups, weights)
    (discrete_ebm.rs:293-359): node groups of equal length (node ids), weights
    of shape [batch, d1, d2] (missing trailing axes are 1)."""

    def __init__(self, spin_node_groups, categorical_node_groups, weights):
        groups = [np.asarray(g.nodes if isinstance(g, Block) else g, np.uint32).reshape(-1)
                  for g in list(spin_node_groups) + list(categorical_node_groups)]
        if not groups:
            raise ThrmlError(_lib.THRML_EINVAL, "At least one node group must be provided")
        n = groups[0].size
        if any(g.size != n for g in groups):
            raise ThrmlError(_lib.THRML_EINVAL,
                             "Every block in node_groups must contain the same number of nodes")
        w = np.asarray(weights, np.float32)
        if w.ndim == 0 or w.ndim > 3:
            raise ThrmlError(_lib.THRML_EINVAL, "weights are [b, d1, d2]")
        if w.shape[0] != n:
            raise ThrmlError(_lib.THRML_EINVAL,
                             "The leading dimension of weights must have the same length as the "
                             "number of nodes in each node group")
        self.n_spin = len(spin_node_groups)
        self.n_cat = len(categorical_node_groups)
        self.nodes = np.ascontiguousarray(np.concatenate(groups))
        self.weights = np.ascontiguousarray(w.reshape(n, *(list(w.shape[1:]) + [1, 1])[:2]))
        self.flags = 0

    @property
    def batch(self):
        return int(self.weights.shape[0])


class SquareDiscreteEBMFactor(DiscreteEBMFactor):
    """SquareDiscreteEBMFactor::new (discrete_ebm.rs:858-1013): weights [b, x, x]
    ("Interaction tensor is not square" otherwise).  Its interaction groups of
    equal (tail count, spin tail count) are merged (merge_interaction_groups,
    :909-986): the two categorical-head groups of a factor with two categorical
    groups are one group, summed together, head group 0's rows first."""

    def __init__(self, spin_node_groups, categorical_node_groups, weights):
        w = np.asarray(weights, np.float32)
        if 0 < w.ndim <= 3:
            dims = (list(w.shape[1:]) + [1, 1])[:2]
            if dims[0] != dims[1]:
                raise ThrmlError(_lib.THRML_EINVAL, "Interaction tensor is not square")
        super().__init__(spin_node_groups, categorical_node_groups, w)
        self.flags = _lib.THRML_FACTOR_SQUARE


def SquareCategoricalEBMFactor(node_groups, weights):
    """SquareCategoricalEBMFactor (discrete_ebm.rs:1014-1064): categorical node
    groups only, weights [b, q, q]."""
    return SquareDiscreteEBMFactor([], node_groups, weights)


def SpinEBMFactor(node_groups, weights):
    """SpinEBMFactor (discrete_ebm.rs): spin node groups only, weights [b, 1, 1]."""
    return DiscreteEBMFactor(node_groups, [], weights)


def CategoricalEBMFactor(node_groups, weights):
    """CategoricalEBMFactor (discrete_ebm.rs): categorical node groups only,
    weights [b, q, 1] or [b, q, q]."""
    return DiscreteEBMFactor([], node_groups, weights)


class FactorSamplingProgram(_Program):
    """FactorSamplingProgram::new (factor.rs:126-185) over DiscreteEBMFactors with
    SpinGibbsConditional on blocks of spin nodes and CategoricalGibbsConditional(q)
    on blocks of categorical nodes.  node_kinds[n] = 0 for a spin node, 1 for a
    categorical node (q categories, 2..65536: one byte of state per node up to
    256, two above; such states read back as uint16).  free_blocks may hold
    superblocks, as for IsingSamplingProgram."""

    def __init__(self, node_kinds, q, factors, free_blocks, clamped_blocks, device):
        self.device = device
        kinds = np.ascontiguousarray(np.asarray(node_kinds, np.uint8).reshape(-1))
        self.q = int(q) if kinds.any() else 2  # q means nothing without categorical nodes
        self.factors = list(factors)
        arr = (_lib.DiscreteFactor * max(len(self.factors), 1))()
        for i, f in enumerate(self.factors):
            arr[i] = _lib.DiscreteFactor(f.n_spin, f.n_cat, f.batch, f.weights.shape[1],
                                         f.weights.shape[2], ptr(f.nodes, ctypes.c_uint32),
                                         ptr(f.weights, ctypes.c_float), f.flags)
        flat, self.sampling_order, sboff = _super_blocks(free_blocks)
        fb, foff, fnodes = _blocks_flat(flat)
        cb, coff, cnodes = _blocks_flat(clamped_blocks)
        self.free_blocks, self.clamped_blocks = fb, cb
        self._keep = (kinds, arr, foff, fnodes, coff, cnodes, sboff)
        d = _lib.DiscreteDesc(kinds.size, ptr(kinds, ctypes.c_uint8), self.q, len(self.factors),
                              ctypes.cast(arr, ctypes.POINTER(_lib.DiscreteFactor)), len(fb),
                              ptr(foff, ctypes.c_uint32), ptr(fnodes, ctypes.c_uint32), len(cb),
                              ptr(coff, ctypes.c_uint32) if cb else None,
                              ptr(cnodes, ctypes.c_uint32) if cb else None,
                              0 if sboff is None else sboff.size - 1, ptr(sboff, ctypes.c_uint32))
        h = ctypes.c_void_p()
        check(load().thrml_discrete_program_create(device.handle, ctypes.byref(d), ctypes.byref(h)))
        self._h = h
        _register(device, self, program=True)


def bf16_round(x):
    """Round float32 to bf16 (nearest even); returns (uint16 bits, float32 values)."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    b = x.view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) >> 16
    bits = b.astype(np.uint16)
    return bits, (bits.astype(np.uint32) << 16).view(np.float32)


class RbmProgram(_Program):
    """Dense bipartite Ising program: visible nodes 0..V-1, hidden V..V+H-1.
    weights [V, H]: uint16 arrays are bf16 bit patterns; any other dtype is
    taken as f32 and held exactly (up to three bf16 pieces per weight, one
    matrix-core pass over K per piece).  clamped=None: blocks [visible,
    hidden], both free; "visible": free [hidden], clamped [visible] (a
    data-clamped positive phase); "hidden": free [visible], clamped
    [hidden]."""

    def __init__(self, weights, bias_visible, bias_hidden, beta, device, clamped=None):
        self.device = device
        W = np.asarray(weights)
        is_bf16 = W.dtype == np.uint16
        W = np.ascontiguousarray(W if is_bf16 else W.astype(np.float32))
        V, H = W.shape
        bv = np.ascontiguousarray(np.asarray(bias_visible, dtype=np.float32).reshape(-1))
        bh = np.ascontiguousarray(np.asarray(bias_hidden, dtype=np.float32).reshape(-1))
        self.V, self.H = int(V), int(H)
        vis, hid = Block(np.arange(V)), Block(np.arange(V, V + H))
        self.free_blocks, self.clamped_blocks = {
            None: ([vis, hid], []), "visible": ([hid], [vis]), "hidden": ([vis], [hid])}[clamped]
        self._keep = (W, bv, bh)
        d = _lib.RbmDesc(V, H, ptr(W, ctypes.c_uint16) if is_bf16 else None,
                         ptr(bv, ctypes.c_float), ptr(bh, ctypes.c_float),
                         float(np.float32(beta)), _lib.RBM_CLAMP[clamped],
                         None if is_bf16 else ptr(W, ctypes.c_float))
        h = ctypes.c_void_p()
        check(load().thrml_rbm_program_create(device.handle, ctypes.byref(d), ctypes.byref(h)))
        self._h = h
        _register(device, self, program=True)

    def half_sweep(self, state, blk, key8):
        key8 = np.ascontiguousarray(np.asarray(key8, dtype=np.uint32).reshape(-1))
        check(load().thrml_rbm_half_sweep(self._h, state._h, int(blk), ptr(key8, ctypes.c_uint32)))


# ---------------------------------------------------------------------------
class DeviceState:
    """n_chains chains resident on the GPU (bit-packed, 64 chains per word)."""

    def __init__(self, program, n_chains):
        self.program = program
        self.n_chains = int(n_chains)
        h = ctypes.c_void_p()
        check(load().thrml_state_create(program._h, self.n_chains, ctypes.byref(h)))
        self._h = h
        _register(program.device, self)

    def set_block(self, b, values):
        _, n = self.program.block_range(b)
        if hasattr(values, "data_ptr"):  # a torch tensor on the device
            import torch
            t = values.contiguous()
            assert t.dtype in (torch.uint8, torch.float32) and t.numel() == self.n_chains * n
            dt = _lib.DTYPE_U8 if t.dtype == torch.uint8 else _lib.DTYPE_F32
            check(load().thrml_state_set_block(self._h, int(b), ctypes.c_void_p(t.data_ptr()), dt,
                                               1 if t.is_cuda else 0))
            return
        a = np.asarray(values)
        if (a.dtype.kind in "biu" and not self._wide and a.size
                and (a.min() < 0 or a.max() > 255)) or a.dtype.kind in "fc" or self._wide:
            # floats, values that a byte cannot hold (which the library then
            # rejects instead of a wrapped byte slipping through) and more
            # than 256 categories cross the C ABI as float32 (exact for every
            # integer below 2^24)
            a = a.astype(np.float32)
            dt = _lib.DTYPE_F32
        else:
            a = a.astype(np.uint8)
            dt = _lib.DTYPE_U8
        a = np.ascontiguousarray(a.reshape(self.n_chains, n))
        check(load().thrml_state_set_block(self._h, int(b), a.ctypes.data, dt, 0))

    @property
    def _wide(self):
        """A categorical program with more than 256 categories (two bytes of
        state per node): uint8 reads become uint16, through float32."""
        return getattr(self.program, "q", 2) > 256

    def get_block(self, b, dtype=np.uint8):
        if self._wide and np.dtype(dtype) != np.float32:
            return self.get_block(b, np.float32).astype(np.uint16)
        _, n = self.program.block_range(b)
        out = np.zeros((self.n_chains, n), dtype=dtype)
        dt = _lib.DTYPE_F32 if out.dtype == np.float32 else _lib.DTYPE_U8
        check(load().thrml_state_get_block(self._h, int(b), out.ctypes.data, dt, 0))
        return out

    def set_global(self, full):
        """full: [n_chains, n_total] in global order (free ++ clamped blocks)."""
        full = np.asarray(full)
        for b in range(len(self.program.free_blocks) + len(self.program.clamped_blocks)):
            off, n = self.program.block_range(b)
            self.set_block(b, np.ascontiguousarray(full[:, off:off + n]))

    def get_global(self):
        out = np.zeros((self.n_chains, self.program.n_total),
                       dtype=np.uint16 if self._wide else np.uint8)
        for b in range(len(self.program.free_blocks) + len(self.program.clamped_blocks)):
            off, n = self.program.block_range(b)
            out[:, off:off + n] = self.get_block(b)
        return out

    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            load().thrml_state_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        # at interpreter exit the HIP runtime may already be gone: leak instead
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:
            pass


def _as_state(program, init_chain_state, state_clamp):
    """Accept a DeviceState, or per-block arrays like the reference."""
    if isinstance(init_chain_state, DeviceState):
        return init_chain_state, False
    blocks = list(init_chain_state)
    c = np.asarray(blocks[0]).reshape(-1, len(program.free_blocks[0])).shape[0]
    st = DeviceState(program, c)
    for b, v in enumerate(blocks):
        st.set_block(b, np.asarray(v).reshape(c, -1))
    for k, v in enumerate(state_clamp or []):
        st.set_block(len(program.free_blocks) + k, np.broadcast_to(
            np.asarray(v).reshape(-1, len(program.clamped_blocks[k])),
            (c, len(program.clamped_blocks[k]))))
    return st, True


def _blocks_out(program, st):
    return [st.get_block(b, np.float32) for b in range(len(program.free_blocks))]


# ---------------------------------------------------------------------------
def hinton_init(key, program, n_chains=None, state=None):
    """hinton_init over the program's free blocks; returns a DeviceState."""
    st = state if state is not None else DeviceState(program, n_chains)
    check(load().thrml_hinton_init(program._h, key.seed, st._h))
    return st


def run_blocks(key, program, init_chain_state, state_clamp=(), n_iters=1, device=None):
    """run_blocks(key, program, init_chain_state, state_clamp, n_iters).

    With a DeviceState the sweep runs in place and the state is returned;
    with per-block arrays, new per-block float32 arrays are returned."""
    st, temp = _as_state(program, init_chain_state, state_clamp)
    check(load().thrml_run_blocks(program._h, key.seed, st._h, int(n_iters)))
    if temp:
        out = _blocks_out(program, st)
        st.close()
        return out
    return st


def _global_positions(program, nodes):
    """Positions in the global state (free blocks, then clamped blocks, each
    at its block_range) of `nodes`: the reference's global location map
    (blockspec.rs:15-67), whose lookup fails for a node in no block."""
    blocks = list(program.free_blocks) + list(program.clamped_blocks)
    owner, where = [], []
    for b, blk in enumerate(blocks):
        off, n = program.block_range(b)
        owner.append(np.asarray(blk.nodes, np.int64))
        where.append(np.arange(off, off + n, dtype=np.int64))
    owner, where = np.concatenate(owner), np.concatenate(where)
    nodes = np.asarray(nodes.nodes if isinstance(nodes, Block) else nodes, np.int64).reshape(-1)
    if nodes.size and nodes.min() < 0:
        raise ThrmlError(_lib.THRML_EINVAL, "Node not found in global location map")
    pos = np.full(max(int(owner.max()), int(nodes.max(initial=0))) + 1, -1, np.int64)
    pos[owner] = where
    p = pos[nodes]
    if (p < 0).any():
        raise ThrmlError(_lib.THRML_EINVAL, "Node not found in global location map")
    return p


def sample_states(key, program, schedule, init_state, state_clamp=(), nodes_to_sample=None,
                  device=None):
    """sample_states (crates/thrml-samplers/src/sampling.rs:128-156).

    With nodes_to_sample (a list of Blocks), one float32 array per block of
    the state values at every observation, [n_samples, len] for one chain as
    the reference's StateObserver stacks them (state_observer.rs:12-50,
    sampling.rs:291-317), [n_samples, n_chains, len] for several.  Without it,
    the whole global state, uint8 [n_samples, n_chains, n_total] (uint16 for
    a categorical program with more than 256 categories)."""
    st, temp = _as_state(program, init_state, state_clamp)
    n_obs = 1 + max(schedule.n_samples - 1, 0)
    if getattr(program, "q", 2) > 256:
        # categories above 255 come back as float32 (exact below 2^24)
        f = np.zeros((n_obs, st.n_chains, program.n_total), dtype=np.float32)
        check(load().thrml_sample_states_as(program._h, key.seed, schedule._c(), st._h,
                                            f.ctypes.data_as(ctypes.c_void_p), _lib.DTYPE_F32))
        out = f.astype(np.uint16)
    else:
        out = np.zeros((n_obs, st.n_chains, program.n_total), dtype=np.uint8)
        check(load().thrml_sample_states(program._h, key.seed, schedule._c(), st._h,
                                         ptr(out, ctypes.c_uint8)))
    c = st.n_chains
    if temp:
        st.close()
    if nodes_to_sample is None:
        return out
    res = []
    for b in nodes_to_sample:
        v = out[:, :, _global_positions(program, b)].astype(np.float32)
        res.append(v[:, 0, :] if c == 1 else v)
    return res


class AbstractObserver:
    """AbstractObserver (crates/thrml-observers/src/observer.rs:9-43):
    init() gives the initial carry; observe(state, carry, iteration) returns
    (carry, observation or None).  `state` is the chains' DeviceState, live
    on the device: read it (get_block, get_global).  Writes to it
    (set_block, set_global, hinton_init) and runs on its device context are
    refused from inside observe with ThrmlError."""

    def init(self):
        return None

    def observe(self, state, carry, iteration):
        raise NotImplementedError


def sample_with_observation(key, program, schedule, init_state, state_clamp=(),
                            observation_carry_init=None, f_observe=None, device=None):
    """sample_with_observation (crates/thrml-samplers/src/sampling.rs:178-320)
    with any AbstractObserver: observe is called after the warm-up
    (iteration 0) and after each further steps_per_sample sweeps (1 ..
    n_samples - 1), from the library's run through a C callback.  Returns
    (final carry, the non-None observations in order).  An exception raised
    in observe stops the run and is raised again here."""
    if f_observe is None:
        raise ValueError("f_observe is required")
    st, temp = _as_state(program, init_state, state_clamp)
    carry = [f_observe.init() if observation_carry_init is None else observation_carry_init]
    observations, error = [], []

    def trampoline(user, iteration, st_ptr, stream):
        try:
            carry[0], obs = f_observe.observe(st, carry[0], int(iteration))
            if obs is not None:
                observations.append(obs)
            return 0
        except BaseException as e:  # re-raised after the library returns
            error.append(e)
            return 1

    cb = _lib.OBSERVE_FN(trampoline)
    try:
        rc = load().thrml_sample_with_observer(program._h, key.seed, schedule._c(), st._h,
                                               ctypes.cast(cb, ctypes.c_void_p), None)
        if error:
            raise error[0]
        check(rc)
    finally:
        if temp:
            st.close()
    return carry[0], observations


class IsingMomentSpec(tuple):
    """(nodes, pairs): the first and second moments of ising_moment_spec."""

    def __new__(cls, nodes, pairs):
        return super().__new__(cls, (nodes, pairs))


def ising_moment_spec(first_moment_nodes, second_moment_edges):
    """(nodes, pairs) of the first and second moments (moment.rs:125-150)."""
    nodes = np.ascontiguousarray(np.asarray(first_moment_nodes, dtype=np.uint32).reshape(-1))
    pairs = np.ascontiguousarray(np.asarray(second_moment_edges, dtype=np.uint32).reshape(-1, 2))
    return IsingMomentSpec(nodes, pairs)


class MomentAccumulatorObserver:
    """MomentAccumulatorObserver::new(moment_spec, transform_to_spin)
    (crates/thrml-observers/src/moment.rs:29-250) bound to one program.

    spec = ising_moment_spec(nodes, edges): sample_with_observation returns the
    exact int64 sums (node_sums, pair_sums); on Ising programs these come from
    the sweep kernels' own counters.  Any other spec is the reference's
    three-level list [moment type][row][nodes]: sample_with_observation then
    returns one int64 array of row sums per moment type, each row the sum over
    chains and observations of prod f(x), f(x) = 2x - 1 with transform_to_spin,
    else x (categories for categorical nodes)."""

    def __init__(self, program, spec, transform_to_spin=True):
        self.program = program
        self._h = None
        self._gen = None
        ising = isinstance(spec, IsingMomentSpec)
        if ising:
            self.nodes, self.pairs = spec
        if ising and transform_to_spin and not isinstance(program, (CategoricalProgram,
                                                                     FactorSamplingProgram)):
            h = ctypes.c_void_p()
            check(load().thrml_moments_create(
                program._h, ptr(self.nodes, ctypes.c_uint32), self.nodes.size,
                ptr(self.pairs, ctypes.c_uint32), self.pairs.shape[0], ctypes.byref(h)))
            self._h = h
        else:
            types = ([[[int(n)] for n in self.nodes], [[int(a), int(b)] for a, b in self.pairs]]
                     if ising else [list(t) for t in spec])
            self._types = [len(t) for t in types]
            rows = [np.asarray(r, np.uint32).reshape(-1) for t in types for r in t]
            off = np.zeros(len(rows) + 1, np.uint64)
            for i, r in enumerate(rows):
                off[i + 1] = off[i] + r.size
            flat = np.ascontiguousarray(np.concatenate(rows) if rows else np.zeros(1, np.uint32))
            h = ctypes.c_void_p()
            check(load().thrml_observer_create(program._h, ptr(off, ctypes.c_uint64), len(rows),
                                               ptr(flat, ctypes.c_uint32),
                                               1 if transform_to_spin else 0, ctypes.byref(h)))
            self._gen = h
            self._ising_split = ising
        _register(program.device, self)

    @property
    def n_nodes(self):
        return int(self.nodes.size)

    @property
    def n_pairs(self):
        return int(self.pairs.shape[0])

    def _run_general(self, key, schedule, state):
        n = sum(self._types)
        sums = np.zeros(max(n, 1), dtype=np.int64)
        check(load().thrml_observer_run(self.program._h, key.seed, schedule._c(), state._h,
                                        self._gen, sums.ctypes.data, 0))
        parts, k = [], 0
        for t in self._types:
            parts.append(sums[k:k + t].copy())
            k += t
        return tuple(parts) if self._ising_split else parts

    def sample_with_observation(self, key, schedule, state, out=None):
        """Runs the schedule on a DeviceState and returns the exact int64 sums
        (node_sums, pair_sums) over chains and observations.  With
        out=(node_tensor, pair_tensor), int64 device tensors, the sums are
        written there on the library stream and nothing is copied to the host."""
        if self._gen is not None:
            res = self._run_general(key, schedule, state)
            if out is not None:
                import torch
                for t, r in zip(out, res):
                    t.copy_(torch.from_numpy(r))
                return out
            return res
        if out is not None:
            a, b = out
            assert a.numel() == self.n_nodes and b.numel() == self.n_pairs
            check(load().thrml_moments_run(self.program._h, key.seed, schedule._c(), state._h,
                                           self._h, ctypes.c_void_p(a.data_ptr()),
                                           ctypes.c_void_p(b.data_ptr()), 1))
            return a, b
        ns = np.zeros(self.n_nodes, dtype=np.int64)
        es = np.zeros(self.n_pairs, dtype=np.int64)
        check(load().thrml_moments_run(self.program._h, key.seed, schedule._c(), state._h,
                                       self._h, ns.ctypes.data, es.ctypes.data, 0))
        return ns, es

    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            load().thrml_moments_destroy(self._h)
            self._h = ctypes.c_void_p()
        if getattr(self, "_gen", None) is not None and self._gen.value:
            load().thrml_observer_destroy(self._gen)
            self._gen = ctypes.c_void_p()

    def __del__(self):
        # at interpreter exit the HIP runtime may already be gone: leak instead
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:
            pass


def estimate_moments(key, first_moment_nodes, second_moment_edges, program, schedule,
                     init_state, clamped_data=(), device=None, return_sums=False,
                     observer=None):
    """estimate_moments (ising.rs:455-505).

    Returns (node_moments, edge_moments) averaged over chains and
    observations: sums / (n_chains * n_samples), as the reference divides its
    single-chain sums by n_samples.  return_sums=True gives the exact int64
    sums over chains and observations instead.  A prebuilt observer for the
    same nodes / edges may be passed to skip the spec construction."""
    st, temp = _as_state(program, init_state, clamped_data)
    own = observer is None
    if own:
        observer = MomentAccumulatorObserver(
            program, ising_moment_spec(first_moment_nodes, second_moment_edges))
    try:
        ns, es = observer.sample_with_observation(key, schedule, st)
    finally:
        if own:
            observer.close()
    c = st.n_chains
    if temp:
        st.close()
    if return_sums:
        return ns, es
    denom = np.float64(c) * schedule.n_samples
    with np.errstate(divide="ignore", invalid="ignore"):
        return ns / denom, es / denom


class IsingTrainingSpec:
    """IsingTrainingSpec::new (crates/thrml-models/src/ising.rs:391-433).

    The positive program samples positive_sampling_blocks with data_blocks and
    then conditioning_blocks clamped; the negative program samples
    negative_sampling_blocks with conditioning_blocks clamped.  dense=True
    runs an RBM's two programs on the matrix cores (IsingSamplingProgram)."""

    def __init__(self, ebm, data_blocks, conditioning_blocks, positive_sampling_blocks,
                 negative_sampling_blocks, schedule_positive, schedule_negative, device=None,
                 dense=False):
        self.ebm = ebm
        self.n_data_blocks = len(data_blocks)
        self.program_positive = IsingSamplingProgram(
            ebm, positive_sampling_blocks, list(data_blocks) + list(conditioning_blocks), device,
            dense=dense)
        self.program_negative = IsingSamplingProgram(
            ebm, negative_sampling_blocks, list(conditioning_blocks), device, dense=dense)
        self.schedule_positive = schedule_positive
        self.schedule_negative = schedule_negative

    def close(self):
        self.program_positive.close()
        self.program_negative.close()


def _n_chains(program, init_state):
    if isinstance(init_state, DeviceState):
        return init_state.n_chains
    return np.asarray(list(init_state)[0]).reshape(-1, len(program.free_blocks[0])).shape[0]


def _phase_means(key, program, schedule, init_state, clamped, bias_nodes, weight_edges):
    """f32 first and second moment means of one phase: int64 sums over chains
    and observations, as f32, divided by chains * n_samples (the reference's
    single-chain carry / n_samples, ising.rs:492-503)."""
    if isinstance(init_state, DeviceState):
        nf = len(program.free_blocks)
        for k, v in enumerate(clamped):
            n = len(program.clamped_blocks[k])
            init_state.set_block(nf + k, np.ascontiguousarray(np.broadcast_to(
                np.asarray(v, np.float32).reshape(-1, n), (init_state.n_chains, n))))
    ns, es = estimate_moments(key, bias_nodes, weight_edges, program, schedule, init_state,
                              clamped, return_sums=True)
    d = np.float32(_n_chains(program, init_state) * schedule.n_samples)
    return ns.astype(np.float32) / d, es.astype(np.float32) / d


def estimate_kl_grad(key, training_spec, bias_nodes, weight_edges, data, conditioning_values,
                     init_state_positive, init_state_negative, device=None):
    """estimate_kl_grad (crates/thrml-models/src/ising.rs:531-595).

    Returns (grad_w, grad_b) = -beta (<.>_+ - <.>_-) in f32.  (key_pos, key_neg)
    = key.split_two().  Positive phase: each data array [batch, n] clamps one
    row per chain, row split(key_pos, C)[c] % batch for chain c of C (for one
    chain, key_pos % batch: the reference's row), followed by the
    conditioning values; negative phase: conditioning values only.  Moments
    are averaged over chains and observations."""
    key_pos, key_neg = key.split_two()
    beta = np.float32(training_spec.ebm.beta)
    sp, sn = training_spec.program_positive, training_spec.program_negative
    chain_keys = key_pos.split(_n_chains(sp, init_state_positive))
    clamped_pos = []
    for d in data:
        d = np.asarray(d, np.float32)
        clamped_pos.append(d[[k.seed % d.shape[0] for k in chain_keys]])
    clamped_pos += [np.asarray(c, np.float32) for c in conditioning_values]
    bp, wp = _phase_means(key_pos, sp, training_spec.schedule_positive, init_state_positive,
                          clamped_pos, bias_nodes, weight_edges)
    bn, wn = _phase_means(key_neg, sn, training_spec.schedule_negative, init_state_negative,
                          [np.asarray(c, np.float32) for c in conditioning_values],
                          bias_nodes, weight_edges)
    return (wp - wn) * -beta, (bp - bn) * -beta


def ising_energy(program, state):
    """IsingEBM::energy_batched (ising.rs:226-320) of every chain of a spin
    program's state: -beta (sum_i b_i s_i + sum_e J_e s_u s_v), f64 [n_chains],
    computed on the device."""
    out = np.zeros(state.n_chains, dtype=np.float64)
    check(load().thrml_ising_energy(program._h, state._h, ptr(out, ctypes.c_double)))
    return out


def potts_energy(program, state):
    """Sum of DiscreteEBMFactor::factor_energy (discrete_ebm.rs:551-593) over a
    categorical program's bias and edge factors for every chain:
    -(sum_n b[n][x_n] + sum_e W[e][x_u][x_v]), f64 [n_chains]."""
    out = np.zeros(state.n_chains, dtype=np.float64)
    check(load().thrml_potts_energy(program._h, state._h, ptr(out, ctypes.c_double)))
    return out


def discrete_energy(program, state):
    """Sum of DiscreteEBMFactor::factor_energy (discrete_ebm.rs:551-593) over a
    FactorSamplingProgram's factors for every chain, f64 [n_chains]."""
    out = np.zeros(state.n_chains, dtype=np.float64)
    check(load().thrml_discrete_energy(program._h, state._h, ptr(out, ctypes.c_double)))
    return out


def energy(program, state):
    """Per-chain energy of a state of any program kind."""
    if isinstance(program, CategoricalProgram):
        return potts_energy(program, state)
    if isinstance(program, FactorSamplingProgram):
        return discrete_energy(program, state)
    return ising_energy(program, state)


# ---------------------------------------------------------------------------
def make_nearest_neighbor_lattice(side_len, torus=True):
    """(n_nodes, edges [E,2], upper Block, lower Block), canonical edge order."""
    lib = load()
    ne = check(lib.thrml_lattice_edges(int(side_len), 1 if torus else 0, None, None))
    u = np.zeros(max(ne, 1), np.uint32)
    v = np.zeros(max(ne, 1), np.uint32)
    check(lib.thrml_lattice_edges(int(side_len), 1 if torus else 0, ptr(u, ctypes.c_uint32),
                                  ptr(v, ctypes.c_uint32)))
    L = (int(side_len) + 1) // 2 * 2
    up = np.zeros(L * L // 2, np.uint32)
    lo = np.zeros(L * L // 2, np.uint32)
    check(lib.thrml_lattice_blocks(int(side_len), ptr(up, ctypes.c_uint32), ptr(lo, ctypes.c_uint32)))
    return L * L, np.stack([u[:ne], v[:ne]], axis=1), Block(up), Block(lo)


def greedy_coloring(n_nodes, edges):
    edges = np.asarray(edges, dtype=np.uint32).reshape(-1, 2)
    u = np.ascontiguousarray(edges[:, 0])
    v = np.ascontiguousarray(edges[:, 1])
    color = np.zeros(max(int(n_nodes), 1), np.uint32)
    check(load().thrml_greedy_coloring(int(n_nodes), u.size, ptr(u, ctypes.c_uint32),
                                       ptr(v, ctypes.c_uint32), ptr(color, ctypes.c_uint32)))
    return color[:int(n_nodes)]


def coloring_to_blocks(color):
    """Blocks in colour order, nodes ascending (lib.rs:186-205)."""
    color = np.asarray(color)
    order = np.argsort(color, kind="stable")
    counts = np.bincount(color)
    out, pos = [], 0
    for c in counts:
        if c:
            out.append(Block(order[pos:pos + c]))
        pos += c
    return out


def erdos_renyi(n_nodes, p, seed):
    lib = load()
    n = check(lib.thrml_erdos_renyi(int(n_nodes), float(p), int(seed), None, None, 0))
    u = np.zeros(max(n, 1), np.uint32)
    v = np.zeros(max(n, 1), np.uint32)
    check(lib.thrml_erdos_renyi(int(n_nodes), float(p), int(seed), ptr(u, ctypes.c_uint32),
                                ptr(v, ctypes.c_uint32), n))
    return np.stack([u[:n], v[:n]], axis=1)


def double_grid(side_len, jumps, n_visible, seed):
    """get_double_grid (crates/thrml-models/tests/test_train_mnist.rs:37-115):
    (upper, lower, visible, upper_without_visible, n_nodes, edges [E, 2]), the
    upper layer nodes 0..side^2, the lower layer side^2..2 side^2, every edge
    (upper, lower)."""
    lib = load()
    j = np.ascontiguousarray(np.asarray(jumps, np.uint32).reshape(-1))
    size = int(side_len) ** 2
    ne = check(lib.thrml_double_grid(int(side_len), ptr(j, ctypes.c_uint32), j.size,
                                     int(n_visible), int(seed), None, None, None))
    u = np.zeros(ne, np.uint32)
    v = np.zeros(ne, np.uint32)
    vis = np.zeros(max(int(n_visible), 1), np.uint32)
    check(lib.thrml_double_grid(int(side_len), ptr(j, ctypes.c_uint32), j.size, int(n_visible),
                                int(seed), ptr(u, ctypes.c_uint32), ptr(v, ctypes.c_uint32),
                                ptr(vis, ctypes.c_uint32)))
    vis = vis[:int(n_visible)]
    rest = np.setdiff1d(np.arange(size, dtype=np.uint32), vis)
    return (Block(np.arange(size, dtype=np.uint32)), Block(np.arange(size, 2 * size, dtype=np.uint32)),
            Block(vis), Block(rest), 2 * size, np.stack([u, v], axis=1))


def param_normal(seed, n, mean, std):
    out = np.zeros(int(n), np.float32)
    check(load().thrml_param_normal(int(seed), int(n), float(mean), float(std),
                                    ptr(out, ctypes.c_float)))
    return out
