// thrml_hip.hpp -- C++ host API of libthrml_hip.so, mirroring thrml-rs's
// sampling API for the block Gibbs path: the same names and argument meanings
// as the reference's Rust functions, with its Result<_, String> error
// convention (Result<T> below).  Header-only C++17 over the C ABI of
// thrml_hip.h; it needs no HIP headers and links only libthrml_hip.so.
//
// Reference interfaces (paths relative to the thrml-rs repository root):
//   RngKey                     crates/thrml-samplers/src/rng.rs:10-44
//   SamplingSchedule           crates/thrml-samplers/src/schedule.rs:4-20
//   Block                      crates/thrml-core/src/block.rs:5
//   IsingEBM                   crates/thrml-models/src/ising.rs:26-143
//   IsingSamplingProgram::new  crates/thrml-models/src/ising.rs:342-388
//   hinton_init                crates/thrml-models/src/ising.rs:602-673
//   run_blocks                 crates/thrml-samplers/src/sampling.rs:81-106
//   sample_states              crates/thrml-samplers/src/sampling.rs:128-156
//   sample_with_observation    crates/thrml-samplers/src/sampling.rs:178-320
//   estimate_moments           crates/thrml-models/src/ising.rs:455-505
//   IsingEBM::energy_batched   crates/thrml-models/src/ising.rs:226-320
//   make_nearest_neighbor_lattice  crates/thrml-models/src/graph_utils.rs:177-243
//   greedy_coloring / coloring_to_blocks  crates/thrml-examples/src/lib.rs:114-205
//
// Differences a caller sees: nodes are indices into the model's node list
// (the reference's Node handles); a State holds n_chains chains (chain c keyed
// by RngKey::split(key, n_chains)[c], so one chain follows the reference's key
// tree exactly) and lives on the device between calls; clamped blocks are
// written into the State (the reference's state_clamp argument).
#pragma once

#include <stdint.h>

#include <algorithm>
#include <exception>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <utility>
#include <vector>

#include "thrml_hip.h"

namespace thrml {

// The error of a failed call: the C ABI's code and message.
struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string &m) : std::runtime_error(m), code(c) {}
};

// Result<T, String>: a value or an error message.  unwrap() returns the value
// or throws Error (where Rust would panic).
template <class T>
class Result {
 public:
  static Result ok(T v) {
    Result r;
    r.ok_ = true;
    r.v_ = std::move(v);
    return r;
  }
  static Result err(int code, std::string msg) {
    Result r;
    r.code_ = code;
    r.msg_ = std::move(msg);
    return r;
  }
  bool is_ok() const { return ok_; }
  bool is_err() const { return !ok_; }
  int code() const { return code_; }
  const std::string &error() const { return msg_; }
  T &unwrap() & {
    if (!ok_) throw Error(code_, msg_);
    return v_;
  }
  T unwrap() && {
    if (!ok_) throw Error(code_, msg_);
    return std::move(v_);
  }

 private:
  bool ok_ = false;
  int code_ = THRML_OK;
  std::string msg_;
  T v_{};
};

template <>
class Result<void> {
 public:
  static Result ok() { return Result(THRML_OK, ""); }
  static Result err(int code, std::string msg) { return Result(code, std::move(msg)); }
  bool is_ok() const { return code_ == THRML_OK; }
  bool is_err() const { return code_ != THRML_OK; }
  int code() const { return code_; }
  const std::string &error() const { return msg_; }
  void unwrap() const {
    if (code_ != THRML_OK) throw Error(code_, msg_);
  }

 private:
  Result(int c, std::string m) : code_(c), msg_(std::move(m)) {}
  int code_;
  std::string msg_;
};

namespace detail {
inline std::string last_error() {
  const char *m = thrml_last_error();
  return m ? std::string(m) : std::string();
}
inline Result<void> check(int rc) {
  return rc == THRML_OK ? Result<void>::ok() : Result<void>::err(rc, last_error());
}
template <class T>
Result<T> fail(int rc) {
  return Result<T>::err(rc, last_error());
}
template <class T>
Result<T> fail(const Result<void> &r) {
  return Result<T>::err(r.code(), r.error());
}
}  // namespace detail

// ---------------------------------------------------------------------------
// RngKey (rng.rs:10-44): split(n) = n x next_u64 of ChaCha8Rng::seed_from_u64,
// bit-exact with the reference's key tree.
class RngKey {
 public:
  explicit RngKey(uint64_t seed) : seed_(seed) {}
  uint64_t seed() const { return seed_; }
  std::vector<RngKey> split(size_t n) const {
    std::vector<uint64_t> k(n ? n : 1);
    if (thrml_rng_split(seed_, n, k.data()) != THRML_OK) throw Error(THRML_EINVAL, detail::last_error());
    std::vector<RngKey> out;
    out.reserve(n);
    for (size_t i = 0; i < n; ++i) out.emplace_back(k[i]);
    return out;
  }
  std::pair<RngKey, RngKey> split_two() const {
    const auto k = split(2);
    return {k[0], k[1]};
  }
  bool operator==(const RngKey &o) const { return seed_ == o.seed_; }

 private:
  uint64_t seed_;
};

// SamplingSchedule (schedule.rs:4-20): n_warmup + (n_samples - 1) *
// steps_per_sample sweeps, n_samples observations (the first after warm-up).
struct SamplingSchedule {
  uint64_t n_warmup, n_samples, steps_per_sample;
  SamplingSchedule(uint64_t w, uint64_t n, uint64_t s) : n_warmup(w), n_samples(n), steps_per_sample(s) {}
  thrml_schedule c() const { return thrml_schedule{n_warmup, n_samples, steps_per_sample}; }
};

// Block (block.rs:5): the nodes of one block, in order.
struct Block {
  std::vector<uint32_t> nodes;
  Block() = default;
  explicit Block(std::vector<uint32_t> n) : nodes(std::move(n)) {}
  size_t len() const { return nodes.size(); }
};

using Edge = std::pair<uint32_t, uint32_t>;

// IsingEBM (ising.rs:26-143): E(s) = -beta (sum_i b_i s_i + sum_(i,j) J_ij s_i s_j).
struct IsingEBM {
  uint32_t n_nodes = 0;
  std::vector<Edge> edges;
  std::vector<float> biases;   // [n_nodes]
  std::vector<float> weights;  // [edges]
  float beta = 1.0f;
};

// ---------------------------------------------------------------------------
// Device: one HIP device and one stream (the reference's WgpuDevice).  Move
// only; programs and states made on it must be destroyed before it.
class Device {
 public:
  static Result<Device> create(int ordinal = 0) {
    thrml_ctx *c = nullptr;
    const int rc = thrml_ctx_create(ordinal, &c);
    if (rc != THRML_OK) return detail::fail<Device>(rc);
    Device d;
    d.ctx_ = c;
    return Result<Device>::ok(std::move(d));
  }
  Device() = default;
  Device(Device &&o) noexcept : ctx_(o.ctx_) { o.ctx_ = nullptr; }
  Device &operator=(Device &&o) noexcept {
    std::swap(ctx_, o.ctx_);
    return *this;
  }
  Device(const Device &) = delete;
  Device &operator=(const Device &) = delete;
  ~Device() {
    if (ctx_) thrml_ctx_destroy(ctx_);
  }
  thrml_ctx *handle() const { return ctx_; }
  Result<void> synchronize() const { return detail::check(thrml_ctx_synchronize(ctx_)); }

 private:
  thrml_ctx *ctx_ = nullptr;
};

// A compiled program (BlockSamplingProgram): immutable, move only.
class Program {
 public:
  Program() = default;
  Program(Program &&o) noexcept : h_(o.h_), free_(std::move(o.free_)), clamped_(std::move(o.clamped_)) {
    o.h_ = nullptr;
  }
  Program &operator=(Program &&o) noexcept {
    std::swap(h_, o.h_);
    std::swap(free_, o.free_);
    std::swap(clamped_, o.clamped_);
    return *this;
  }
  Program(const Program &) = delete;
  Program &operator=(const Program &) = delete;
  ~Program() {
    if (h_) thrml_prog_destroy(h_);
  }
  thrml_prog *handle() const { return h_; }
  // 0 Ising lattice, 1 Ising CSR, 2 categorical, 3 dense bipartite
  uint32_t kind() const { return info().kind; }
  uint64_t n_total() const { return info().n_total; }
  const std::vector<Block> &free_blocks() const { return free_; }
  const std::vector<Block> &clamped_blocks() const { return clamped_; }
  // (global offset, length) of block b: free blocks first, then clamped
  std::pair<uint64_t, uint64_t> block_range(uint32_t b) const {
    uint64_t off = 0, len = 0;
    if (thrml_prog_block(h_, b, &off, &len) != THRML_OK) throw Error(THRML_EINVAL, detail::last_error());
    return {off, len};
  }

 protected:
  thrml_prog_info info() const {
    thrml_prog_info i{};
    thrml_prog_get_info(h_, &i);
    return i;
  }
  static void flatten(const std::vector<Block> &bs, std::vector<uint32_t> &off, std::vector<uint32_t> &nodes) {
    off.assign(1, 0);
    nodes.clear();
    for (const Block &b : bs) {
      nodes.insert(nodes.end(), b.nodes.begin(), b.nodes.end());
      off.push_back((uint32_t)nodes.size());
    }
  }
  thrml_prog *h_ = nullptr;
  std::vector<Block> free_, clamped_;
};

// IsingSamplingProgram::new(ebm, free_blocks, clamped_blocks, device)
// (ising.rs:342-388): SpinGibbsConditional on every free block, each its own
// superblock unless superblock_offsets groups them (offsets over the free
// blocks, BlockGibbsSpec::new, program.rs:28-64).  flags = THRML_ISING_DENSE
// sends a complete bipartite model (an RBM) to the matrix cores, whose f32
// summation order may flip decisions at threshold sites.
class IsingSamplingProgram : public Program {
 public:
  static Result<IsingSamplingProgram> create(const IsingEBM &ebm, const std::vector<Block> &free_blocks,
                                             const std::vector<Block> &clamped_blocks, Device &dev,
                                             const std::vector<uint32_t> &superblock_offsets = {},
                                             uint32_t flags = 0) {
    std::vector<uint32_t> eu(ebm.edges.size()), ev(ebm.edges.size());
    for (size_t e = 0; e < ebm.edges.size(); ++e) {
      eu[e] = ebm.edges[e].first;
      ev[e] = ebm.edges[e].second;
    }
    if (ebm.biases.size() != ebm.n_nodes || ebm.weights.size() != ebm.edges.size())
      return Result<IsingSamplingProgram>::err(THRML_EINVAL, "biases / weights do not match nodes / edges");
    std::vector<uint32_t> fo, fn, co, cn;
    flatten(free_blocks, fo, fn);
    flatten(clamped_blocks, co, cn);
    thrml_ising_desc d{};
    d.n_nodes = ebm.n_nodes;
    d.n_edges = ebm.edges.size();
    d.edge_u = eu.data();
    d.edge_v = ev.data();
    d.biases = ebm.biases.data();
    d.weights = ebm.weights.data();
    d.beta = ebm.beta;
    d.n_free_blocks = (uint32_t)free_blocks.size();
    d.free_offsets = fo.data();
    d.free_nodes = fn.data();
    d.n_clamped_blocks = (uint32_t)clamped_blocks.size();
    d.clamped_offsets = clamped_blocks.empty() ? nullptr : co.data();
    d.clamped_nodes = clamped_blocks.empty() ? nullptr : cn.data();
    d.n_superblocks = superblock_offsets.empty() ? 0u : (uint32_t)superblock_offsets.size() - 1u;
    d.superblock_offsets = superblock_offsets.empty() ? nullptr : superblock_offsets.data();
    d.flags = flags;
    IsingSamplingProgram p;
    const int rc = thrml_ising_program_create(dev.handle(), &d, &p.h_);
    if (rc != THRML_OK) return detail::fail<IsingSamplingProgram>(rc);
    p.free_ = free_blocks;
    p.clamped_ = clamped_blocks;
    return Result<IsingSamplingProgram>::ok(std::move(p));
  }
};

// A categorical (Potts) program: bias factor b[N][q] and edge factor
// CategoricalEBMFactor([U, V], W[E][q][q]), CategoricalGibbsConditional(q, 0)
// on every free block (discrete_ebm.rs:456-548, softmax.rs:228-271);
// superblock_offsets as for IsingSamplingProgram.
class CategoricalProgram : public Program {
 public:
  static Result<CategoricalProgram> create(uint32_t n_nodes, uint32_t q, const std::vector<Edge> &edges,
                                           const std::vector<float> &weights, const std::vector<float> &biases,
                                           const std::vector<Block> &free_blocks, Device &dev,
                                           const std::vector<Block> &clamped_blocks = {},
                                           const std::vector<uint32_t> &superblock_offsets = {}) {
    if (weights.size() != edges.size() * q * q || biases.size() != (size_t)n_nodes * q)
      return Result<CategoricalProgram>::err(THRML_EINVAL, "weights / biases do not match edges / nodes");
    std::vector<uint32_t> eu(edges.size()), ev(edges.size()), fo, fn, co, cn;
    for (size_t e = 0; e < edges.size(); ++e) {
      eu[e] = edges[e].first;
      ev[e] = edges[e].second;
    }
    flatten(free_blocks, fo, fn);
    flatten(clamped_blocks, co, cn);
    thrml_potts_desc d{};
    d.n_nodes = n_nodes;
    d.q = q;
    d.n_edges = edges.size();
    d.edge_u = eu.data();
    d.edge_v = ev.data();
    d.weights = weights.data();
    d.biases = biases.data();
    d.n_free_blocks = (uint32_t)free_blocks.size();
    d.free_offsets = fo.data();
    d.free_nodes = fn.data();
    d.n_clamped_blocks = (uint32_t)clamped_blocks.size();
    d.clamped_offsets = clamped_blocks.empty() ? nullptr : co.data();
    d.clamped_nodes = clamped_blocks.empty() ? nullptr : cn.data();
    d.n_superblocks = superblock_offsets.empty() ? 0u : (uint32_t)superblock_offsets.size() - 1u;
    d.superblock_offsets = superblock_offsets.empty() ? nullptr : superblock_offsets.data();
    CategoricalProgram p;
    const int rc = thrml_potts_program_create(dev.handle(), &d, &p.h_);
    if (rc != THRML_OK) return detail::fail<CategoricalProgram>(rc);
    p.free_ = free_blocks;
    p.clamped_ = clamped_blocks;
    return Result<CategoricalProgram>::ok(std::move(p));
  }
};

// DiscreteEBMFactor (discrete_ebm.rs:293-359): spin node groups, then up to
// two categorical node groups, of equal length; weights [batch][d1][d2].
// square = true: SquareDiscreteEBMFactor (discrete_ebm.rs:858-1013), d1 == d2,
// its two categorical-head interaction groups merged.
struct DiscreteFactor {
  std::vector<Block> spin_groups, cat_groups;
  std::vector<float> weights;
  uint32_t d1 = 1, d2 = 1;
  bool square = false;
};

// FactorSamplingProgram::new (factor.rs:126-185) over discrete factors:
// SpinGibbsConditional on blocks of spin nodes, CategoricalGibbsConditional(q)
// on blocks of categorical nodes.  node_kind[n] = 0 spin, 1 categorical.
class FactorSamplingProgram : public Program {
 public:
  static Result<FactorSamplingProgram> create(const std::vector<uint8_t> &node_kind, uint32_t q,
                                              const std::vector<DiscreteFactor> &factors,
                                              const std::vector<Block> &free_blocks, Device &dev,
                                              const std::vector<Block> &clamped_blocks = {},
                                              const std::vector<uint32_t> &superblock_offsets = {}) {
    std::vector<std::vector<uint32_t>> nodes(factors.size());
    std::vector<thrml_discrete_factor> fs(factors.size());
    for (size_t i = 0; i < factors.size(); ++i) {
      const DiscreteFactor &f = factors[i];
      const size_t batch = f.spin_groups.empty() ? (f.cat_groups.empty() ? 0 : f.cat_groups[0].len())
                                                 : f.spin_groups[0].len();
      for (const auto *gs : {&f.spin_groups, &f.cat_groups})
        for (const Block &g : *gs) {
          if (g.len() != batch)
            return Result<FactorSamplingProgram>::err(
                THRML_EINVAL, "Every block in node_groups must contain the same number of nodes");
          nodes[i].insert(nodes[i].end(), g.nodes.begin(), g.nodes.end());
        }
      if (f.weights.size() != batch * f.d1 * f.d2)
        return Result<FactorSamplingProgram>::err(
            THRML_EINVAL,
            "The leading dimension of weights must have the same length as the number of nodes in "
            "each node group");
      fs[i] = thrml_discrete_factor{(uint32_t)f.spin_groups.size(), (uint32_t)f.cat_groups.size(),
                                    (uint32_t)batch, f.d1, f.d2, nodes[i].data(), f.weights.data(),
                                    f.square ? THRML_FACTOR_SQUARE : 0u};
    }
    std::vector<uint32_t> fo, fn, co, cn;
    flatten(free_blocks, fo, fn);
    flatten(clamped_blocks, co, cn);
    thrml_discrete_desc d{};
    d.n_nodes = (uint32_t)node_kind.size();
    d.node_kind = node_kind.data();
    d.q = q;
    d.n_factors = (uint32_t)fs.size();
    d.factors = fs.data();
    d.n_free_blocks = (uint32_t)free_blocks.size();
    d.free_offsets = fo.data();
    d.free_nodes = fn.data();
    d.n_clamped_blocks = (uint32_t)clamped_blocks.size();
    d.clamped_offsets = clamped_blocks.empty() ? nullptr : co.data();
    d.clamped_nodes = clamped_blocks.empty() ? nullptr : cn.data();
    d.n_superblocks = superblock_offsets.empty() ? 0u : (uint32_t)superblock_offsets.size() - 1u;
    d.superblock_offsets = superblock_offsets.empty() ? nullptr : superblock_offsets.data();
    FactorSamplingProgram p;
    const int rc = thrml_discrete_program_create(dev.handle(), &d, &p.h_);
    if (rc != THRML_OK) return detail::fail<FactorSamplingProgram>(rc);
    p.free_ = free_blocks;
    p.clamped_ = clamped_blocks;
    return Result<FactorSamplingProgram>::ok(std::move(p));
  }
};

// Round f32 to bf16 (nearest even): a bf16 RBM's weights, and the first of
// the pieces a dense program holds an f32 weight as.
inline uint16_t bf16_round(float x) {
  uint32_t b;
  static_assert(sizeof b == sizeof x, "");
  __builtin_memcpy(&b, &x, 4);
  return (uint16_t)((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

// A dense bipartite IsingEBM (an RBM: visible nodes 0..V-1, hidden nodes
// V..V+H-1, edge (v, V+h) of f32 weight W[v][h], held exactly as up to three
// bf16 pieces), run on the matrix cores.  clamped = THRML_RBM_CLAMP_NONE: blocks [visible, hidden],
// both free; THRML_RBM_CLAMP_VISIBLE: free [hidden], clamped [visible];
// THRML_RBM_CLAMP_HIDDEN: free [visible], clamped [hidden].
class RbmProgram : public Program {
 public:
  static Result<RbmProgram> create(uint32_t V, uint32_t H, const std::vector<float> &W,
                                   const std::vector<float> &bv, const std::vector<float> &bh, float beta,
                                   Device &dev, uint32_t clamped = THRML_RBM_CLAMP_NONE) {
    if (W.size() != (size_t)V * H || bv.size() != V || bh.size() != H)
      return Result<RbmProgram>::err(THRML_EINVAL, "weights / biases do not match V x H");
    thrml_rbm_desc d{V, H, nullptr, bv.data(), bh.data(), beta, clamped, W.data()};
    RbmProgram p;
    const int rc = thrml_rbm_program_create(dev.handle(), &d, &p.h_);
    if (rc != THRML_OK) return detail::fail<RbmProgram>(rc);
    std::vector<uint32_t> a(V), b(H);
    for (uint32_t i = 0; i < V; ++i) a[i] = i;
    for (uint32_t i = 0; i < H; ++i) b[i] = V + i;
    if (clamped == THRML_RBM_CLAMP_VISIBLE) {
      p.free_ = {Block(b)};
      p.clamped_ = {Block(a)};
    } else if (clamped == THRML_RBM_CLAMP_HIDDEN) {
      p.free_ = {Block(a)};
      p.clamped_ = {Block(b)};
    } else {
      p.free_ = {Block(a), Block(b)};
    }
    return Result<RbmProgram>::ok(std::move(p));
  }
};

// ---------------------------------------------------------------------------
// n_chains chains resident on the device.  Blocks are read and written as
// [n_chains][block_len], f32 0.0/1.0 (or a category index) as the reference
// holds them, or u8; the global state is [n_chains][n_total] u8.
class State {
 public:
  static Result<State> create(Program &prog, uint32_t n_chains) {
    State s;
    const int rc = thrml_state_create(prog.handle(), n_chains, &s.h_);
    if (rc != THRML_OK) return detail::fail<State>(rc);
    s.prog_ = &prog;
    s.C_ = n_chains;
    return Result<State>::ok(std::move(s));
  }
  State() = default;
  State(State &&o) noexcept : h_(o.h_), prog_(o.prog_), C_(o.C_) { o.h_ = nullptr; }
  State &operator=(State &&o) noexcept {
    std::swap(h_, o.h_);
    std::swap(prog_, o.prog_);
    std::swap(C_, o.C_);
    return *this;
  }
  State(const State &) = delete;
  State &operator=(const State &) = delete;
  ~State() {
    if (h_) thrml_state_destroy(h_);
  }
  thrml_state *handle() const { return h_; }
  uint32_t n_chains() const { return C_; }

  Result<void> set_block(uint32_t b, const std::vector<float> &v) {
    if (v.size() != (size_t)C_ * prog_->block_range(b).second)
      return Result<void>::err(THRML_EINVAL, "block data has the wrong size");
    return detail::check(thrml_state_set_block(h_, b, v.data(), THRML_DTYPE_F32, 0));
  }
  Result<std::vector<float>> get_block(uint32_t b) const {
    std::vector<float> v((size_t)C_ * prog_->block_range(b).second);
    const int rc = thrml_state_get_block(h_, b, v.data(), THRML_DTYPE_F32, 0);
    if (rc != THRML_OK) return detail::fail<std::vector<float>>(rc);
    return Result<std::vector<float>>::ok(std::move(v));
  }
  // The whole state [n_chains][n_total] in global order, one byte per node.
  Result<void> set_global(const std::vector<uint8_t> &g) { return set_global_as<uint8_t>(g); }
  Result<std::vector<uint8_t>> get_global() const { return get_global_as<uint8_t>(); }
  // The same with two bytes per node, for programs with more than 256
  // categories (through f32 blocks, exact for every category).
  Result<void> set_global16(const std::vector<uint16_t> &g) { return set_global_as<uint16_t>(g); }
  Result<std::vector<uint16_t>> get_global16() const { return get_global_as<uint16_t>(); }

 private:
  // blocks cross the C ABI as u8 for byte values, as f32 otherwise
  template <class T>
  Result<void> set_global_as(const std::vector<T> &g) {
    constexpr int dt = sizeof(T) == 1 ? THRML_DTYPE_U8 : THRML_DTYPE_F32;
    using E = typename std::conditional<sizeof(T) == 1, uint8_t, float>::type;
    const uint64_t nt = prog_->n_total();
    if (g.size() != (size_t)C_ * nt) return Result<void>::err(THRML_EINVAL, "state has the wrong size");
    const uint32_t nb = (uint32_t)(prog_->free_blocks().size() + prog_->clamped_blocks().size());
    for (uint32_t b = 0; b < nb; ++b) {
      const auto r = prog_->block_range(b);
      std::vector<E> blk((size_t)C_ * r.second);
      for (uint32_t c = 0; c < C_; ++c)
        for (uint64_t i = 0; i < r.second; ++i) blk[(size_t)c * r.second + i] = (E)g[(size_t)c * nt + r.first + i];
      const auto rc = detail::check(thrml_state_set_block(h_, b, blk.data(), dt, 0));
      if (rc.is_err()) return rc;
    }
    return Result<void>::ok();
  }
  template <class T>
  Result<std::vector<T>> get_global_as() const {
    constexpr int dt = sizeof(T) == 1 ? THRML_DTYPE_U8 : THRML_DTYPE_F32;
    using E = typename std::conditional<sizeof(T) == 1, uint8_t, float>::type;
    const uint64_t nt = prog_->n_total();
    std::vector<T> g((size_t)C_ * nt);
    const uint32_t nb = (uint32_t)(prog_->free_blocks().size() + prog_->clamped_blocks().size());
    for (uint32_t b = 0; b < nb; ++b) {
      const auto r = prog_->block_range(b);
      std::vector<E> blk((size_t)C_ * r.second);
      const int rc = thrml_state_get_block(h_, b, blk.data(), dt, 0);
      if (rc != THRML_OK) return detail::fail<std::vector<T>>(rc);
      for (uint32_t c = 0; c < C_; ++c)
        for (uint64_t i = 0; i < r.second; ++i) g[(size_t)c * nt + r.first + i] = (T)blk[(size_t)c * r.second + i];
    }
    return Result<std::vector<T>>::ok(std::move(g));
  }

  thrml_state *h_ = nullptr;
  Program *prog_ = nullptr;
  uint32_t C_ = 0;
};

// hinton_init(key, model, blocks, batch_shape, device) (ising.rs:602-673):
// a new state of n_chains chains with every free block initialised.
inline Result<State> hinton_init(const RngKey &key, Program &prog, uint32_t n_chains) {
  auto st = State::create(prog, n_chains);
  if (st.is_err()) return st;
  const int rc = thrml_hinton_init(prog.handle(), key.seed(), st.unwrap().handle());
  if (rc != THRML_OK) return detail::fail<State>(rc);
  return st;
}

// run_blocks(key, program, state, clamp, n_iters, device) (sampling.rs:81-106):
// n_iters sweeps in place (n_iters = 0 leaves the state unchanged).
inline Result<void> run_blocks(const RngKey &key, Program &prog, State &st, uint64_t n_iters) {
  return detail::check(thrml_run_blocks(prog.handle(), key.seed(), st.handle(), n_iters));
}

// estimate_moments(key, nodes, edges, program, schedule, init, clamp, device)
// (ising.rs:455-505): <s_i> and <s_i s_j> with s = 2x - 1, averaged over the
// chains and the n_samples observations (the reference averages one chain's
// observations); the exact integer sums as well.
struct Moments {
  std::vector<double> nodes, edges;
  std::vector<int64_t> node_sums, edge_sums;
};
inline Result<Moments> estimate_moments(const RngKey &key, const std::vector<uint32_t> &nodes,
                                        const std::vector<Edge> &edges, Program &prog,
                                        const SamplingSchedule &sched, State &st) {
  std::vector<uint32_t> pairs(2 * edges.size());
  for (size_t e = 0; e < edges.size(); ++e) {
    pairs[2 * e] = edges[e].first;
    pairs[2 * e + 1] = edges[e].second;
  }
  Moments m;
  m.node_sums.assign(std::max<size_t>(nodes.size(), 1), 0);
  m.edge_sums.assign(std::max<size_t>(edges.size(), 1), 0);
  const int rc = thrml_estimate_moments(prog.handle(), key.seed(), sched.c(), st.handle(), nodes.data(),
                                        nodes.size(), pairs.data(), edges.size(), m.node_sums.data(),
                                        m.edge_sums.data());
  if (rc != THRML_OK) return detail::fail<Moments>(rc);
  m.node_sums.resize(nodes.size());
  m.edge_sums.resize(edges.size());
  const double n = (double)st.n_chains() * (double)std::max<uint64_t>(sched.n_samples, 1);
  for (int64_t s : m.node_sums) m.nodes.push_back((double)s / n);
  for (int64_t s : m.edge_sums) m.edges.push_back((double)s / n);
  return Result<Moments>::ok(std::move(m));
}

// sample_states(key, program, schedule, init, clamp, nodes, device)
// (sampling.rs:128-156) for the whole global state: [n_obs][n_chains][n_total].
inline Result<std::vector<uint8_t>> sample_states(const RngKey &key, Program &prog,
                                                  const SamplingSchedule &sched, State &st) {
  const uint64_t n_obs = std::max<uint64_t>(sched.n_samples, 1);
  std::vector<uint8_t> out((size_t)n_obs * st.n_chains() * prog.n_total());
  const int rc = thrml_sample_states(prog.handle(), key.seed(), sched.c(), st.handle(), out.data());
  if (rc != THRML_OK) return detail::fail<std::vector<uint8_t>>(rc);
  return Result<std::vector<uint8_t>>::ok(std::move(out));
}

// The same in the StateObserver's f32 representation (state_observer.rs:12-50),
// which also holds categories above 255.
inline Result<std::vector<float>> sample_states_f32(const RngKey &key, Program &prog,
                                                    const SamplingSchedule &sched, State &st) {
  const uint64_t n_obs = std::max<uint64_t>(sched.n_samples, 1);
  std::vector<float> out((size_t)n_obs * st.n_chains() * prog.n_total());
  const int rc = thrml_sample_states_as(prog.handle(), key.seed(), sched.c(), st.handle(),
                                        out.data(), THRML_DTYPE_F32);
  if (rc != THRML_OK) return detail::fail<std::vector<float>>(rc);
  return Result<std::vector<float>>::ok(std::move(out));
}

// sample_with_observation(key, program, schedule, init, clamp, carry_init,
// f_observe) (sampling.rs:178-320) with any observer: a callable
//   int observe(uint64_t iteration, State &state, void *hip_stream)
// in the place of AbstractObserver::observe (crates/thrml-observers/src/
// observer.rs:9-43), called after the warm-up (iteration 0) and after each
// further steps_per_sample sweeps; its carry lives in the callable.  It reads
// the state and may queue work on hip_stream; a nonzero return stops the run.
// An exception thrown by the callable stops the run too (it does not cross
// the C ABI) and is thrown again from here once the run has ended.
template <class F>
inline Result<bool> sample_with_observation(const RngKey &key, Program &prog,
                                            const SamplingSchedule &sched, State &st, F &&observe) {
  struct Call {
    std::remove_reference_t<F> *f;
    State *st;
    std::exception_ptr err;
  } call{&observe, &st, nullptr};
  const thrml_observe_fn tramp = [](void *user, uint64_t iteration, thrml_state *, void *stream) -> int {
    Call *c = static_cast<Call *>(user);
    try {
      return (*c->f)(iteration, *c->st, stream);
    } catch (...) {
      c->err = std::current_exception();
      return THRML_EINVAL;
    }
  };
  const int rc = thrml_sample_with_observer(prog.handle(), key.seed(), sched.c(), st.handle(), tramp, &call);
  if (call.err) std::rethrow_exception(call.err);
  if (rc != THRML_OK) return detail::fail<bool>(rc);
  return Result<bool>::ok(true);
}

// IsingEBM::energy_batched (ising.rs:226-320) of every chain (spin programs),
// or the summed factor energies (categorical and discrete factor programs).
inline Result<std::vector<double>> energy(Program &prog, State &st) {
  std::vector<double> e(st.n_chains());
  const int rc = prog.kind() == 2   ? thrml_potts_energy(prog.handle(), st.handle(), e.data())
                 : prog.kind() == 4 ? thrml_discrete_energy(prog.handle(), st.handle(), e.data())
                                    : thrml_ising_energy(prog.handle(), st.handle(), e.data());
  if (rc != THRML_OK) return detail::fail<std::vector<double>>(rc);
  return Result<std::vector<double>>::ok(std::move(e));
}

// ---------------------------------------------------------------------------
// Graph builders (canonical deterministic orders).
struct Lattice {
  uint32_t n_nodes;
  std::vector<Edge> edges;
  Block upper, lower;  // (i + j) even, odd (graph_utils.rs:232)
};
inline Lattice make_nearest_neighbor_lattice(uint32_t side, bool torus = true) {
  const int64_t ne = thrml_lattice_edges(side, torus ? 1 : 0, nullptr, nullptr);
  if (ne < 0) throw Error((int)ne, detail::last_error());
  std::vector<uint32_t> u(ne), v(ne);
  thrml_lattice_edges(side, torus ? 1 : 0, u.data(), v.data());
  const uint32_t s = side + (side & 1u);
  Lattice L;
  L.n_nodes = s * s;
  for (int64_t e = 0; e < ne; ++e) L.edges.emplace_back(u[e], v[e]);
  std::vector<uint32_t> up(L.n_nodes / 2), lo(L.n_nodes / 2);
  if (thrml_lattice_blocks(side, up.data(), lo.data()) != THRML_OK) throw Error(THRML_EINVAL, detail::last_error());
  L.upper = Block(up);
  L.lower = Block(lo);
  return L;
}

// greedy_coloring (lib.rs:114-147): smallest free colour in node order.
inline std::vector<uint32_t> greedy_coloring(uint32_t n_nodes, const std::vector<Edge> &edges) {
  std::vector<uint32_t> u(edges.size()), v(edges.size()), color(n_nodes);
  for (size_t e = 0; e < edges.size(); ++e) {
    u[e] = edges[e].first;
    v[e] = edges[e].second;
  }
  if (thrml_greedy_coloring(n_nodes, edges.size(), u.data(), v.data(), color.data()) < 0)
    throw Error(THRML_EINVAL, detail::last_error());
  return color;
}

// coloring_to_blocks (lib.rs:186-205): one block per used colour, in colour
// order, nodes ascending.
inline std::vector<Block> coloring_to_blocks(const std::vector<uint32_t> &color) {
  uint32_t k = 0;
  for (uint32_t c : color) k = std::max(k, c + 1);
  std::vector<Block> blocks(k);
  for (uint32_t i = 0; i < color.size(); ++i) blocks[color[i]].nodes.push_back(i);
  blocks.erase(std::remove_if(blocks.begin(), blocks.end(), [](const Block &b) { return b.nodes.empty(); }),
               blocks.end());
  return blocks;
}

}  // namespace thrml
