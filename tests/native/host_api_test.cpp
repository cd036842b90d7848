// host_api_test.cpp -- the C++ host API (include/thrml_hip.hpp) exercised the
// way the reference's own tests exercise thrml-rs, with the CPU oracle
// (oracle/, test infrastructure) as the checker for the sampled states.
//
//   host_api_test            every case (needs a GPU)
//   host_api_test --cpu-only only the cases that make no GPU call
//
// Prints PASS / FAIL per case and exits non-zero on any failure.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <memory>
#include <random>
#include <set>
#include <string>
#include <vector>

#include "../../include/thrml_hip.hpp"
#include "../../oracle/thrml_oracle.h"

using namespace thrml;

namespace {

int g_fail = 0;  // failed checks in the current case

#define CHECK(cond)                                                             \
  do {                                                                          \
    if (!(cond)) {                                                              \
      std::printf("  check failed: %s (%s:%d)\n", #cond, __FILE__, __LINE__);   \
      ++g_fail;                                                                 \
    }                                                                           \
  } while (0)

std::vector<float> normal(uint64_t seed, size_t n, double mean, double std) {
  std::vector<float> v(n ? n : 1);
  thrml_param_normal(seed, n, mean, std, v.data());
  v.resize(n);
  return v;
}

// an oracle program for the same model and blocks
struct OracleIsing {
  orc_ising *p = nullptr;
  OracleIsing(const IsingEBM &ebm, const std::vector<Block> &fb, const std::vector<Block> &cb) {
    std::vector<uint32_t> eu, ev, fo{0}, fn, co{0}, cn;
    for (const Edge &e : ebm.edges) {
      eu.push_back(e.first);
      ev.push_back(e.second);
    }
    for (const Block &b : fb) {
      fn.insert(fn.end(), b.nodes.begin(), b.nodes.end());
      fo.push_back((uint32_t)fn.size());
    }
    for (const Block &b : cb) {
      cn.insert(cn.end(), b.nodes.begin(), b.nodes.end());
      co.push_back((uint32_t)cn.size());
    }
    char err[256];
    p = orc_ising_create(ebm.n_nodes, ebm.edges.size(), eu.data(), ev.data(), ebm.biases.data(),
                         ebm.weights.data(), ebm.beta, (uint32_t)fb.size(), fo.data(), fn.data(),
                         (uint32_t)cb.size(), co.data(), cn.data(), err, sizeof err);
  }
  ~OracleIsing() { orc_ising_destroy(p); }
};

IsingEBM lattice_ebm(uint32_t side, double b_std, double j_mean, double j_std, float beta,
                     std::vector<Block> &blocks) {
  Lattice L = make_nearest_neighbor_lattice(side, true);
  IsingEBM ebm;
  ebm.n_nodes = L.n_nodes;
  ebm.edges = L.edges;
  ebm.biases = normal(1001, L.n_nodes, 0.0, b_std);
  ebm.weights = normal(1101, L.edges.size(), j_mean, j_std);
  ebm.beta = beta;
  blocks = {L.upper, L.lower};
  return ebm;
}

std::vector<Edge> random_edges(uint32_t n, size_t m, uint64_t seed) {
  std::mt19937_64 rng(seed);
  std::set<Edge> s;
  while (s.size() < m) {
    const uint32_t a = (uint32_t)(rng() % n), b = (uint32_t)(rng() % n);
    if (a != b) s.insert({a, b});  // either orientation
  }
  return std::vector<Edge>(s.begin(), s.end());
}

// ---- cases without GPU calls --------------------------------------------
// crates/thrml-samplers/src/rng.rs:57-86, plus bit-exactness with the oracle
void rng_split() {
  const RngKey k(42);
  CHECK(k.split(0).empty());
  CHECK(k.split(1).size() == 1 && k.split(1)[0] == k);
  const auto ten = k.split(10);
  std::set<uint64_t> u;
  for (const RngKey &x : ten) u.insert(x.seed());
  CHECK(u.size() == 10);
  CHECK(k.split(10) == ten);
  const auto two = k.split_two();
  CHECK(two.first == ten[0] && two.second == RngKey(k.split(2)[1]));
  for (uint64_t key : {0ull, 1ull, 42ull, 0xdeadbeefcafef00dull}) {
    std::vector<uint64_t> o(7);
    orc_rng_split(key, 7, o.data());
    const auto s = RngKey(key).split(7);
    for (int i = 0; i < 7; ++i) CHECK(s[i].seed() == o[i]);
  }
}

// crates/thrml-models/src/graph_utils.rs:306-328 (24 / 32 edges on 4 x 4)
void lattice_graph() {
  const Lattice t = make_nearest_neighbor_lattice(4, true), o = make_nearest_neighbor_lattice(4, false);
  CHECK(t.n_nodes == 16 && t.edges.size() == 32);
  CHECK(o.edges.size() == 24);
  CHECK(t.upper.len() == 8 && t.lower.len() == 8);
  for (uint32_t x : t.upper.nodes) CHECK(((x / 4) + (x % 4)) % 2 == 0);  // (i + j) even
  for (const Edge &e : t.edges) CHECK(e.first < e.second);
}

// crates/thrml-examples/src/lib.rs:247-302 (a chain takes 2 colours; a
// bipartite graph is coloured by its sides)
void coloring() {
  const std::vector<Edge> chain{{0, 1}, {1, 2}, {2, 3}, {3, 4}};
  const auto c = greedy_coloring(5, chain);
  CHECK((c == std::vector<uint32_t>{0, 1, 0, 1, 0}));
  const auto blocks = coloring_to_blocks(c);
  CHECK(blocks.size() == 2 && blocks[0].nodes == (std::vector<uint32_t>{0, 2, 4}));
  std::vector<Edge> kb;
  for (uint32_t a = 0; a < 2; ++a)
    for (uint32_t b = 2; b < 5; ++b) kb.push_back({a, b});
  const auto cb = greedy_coloring(5, kb);
  CHECK(cb[0] == cb[1] && cb[2] == cb[3] && cb[3] == cb[4] && cb[0] != cb[2]);
}

// ---- GPU cases ------------------------------------------------------------
// crates/thrml-models/tests/test_ising.rs:139-212 (values worked by hand)
void energy_reference_cases(Device &dev) {
  IsingEBM ebm{3, {{0, 1}, {1, 2}}, {0.1f, 0.2f, 0.3f}, {0.5f, -0.5f}, 1.0f};
  auto prog = IsingSamplingProgram::create(ebm, {Block({0, 1, 2})}, {}, dev).unwrap();
  auto st = State::create(prog, 4).unwrap();
  st.set_global({0, 0, 0, 1, 1, 1, 1, 0, 1, 0, 1, 0}).unwrap();
  const auto e = energy(prog, st).unwrap();
  const double want[4] = {0.6, -0.6, -0.2, 0.2};
  for (int c = 0; c < 4; ++c) CHECK(std::fabs(e[c] - want[c]) < 1e-6);
  IsingEBM chain{4, {{0, 1}, {1, 2}, {2, 3}}, {0, 0, 0, 0}, {1, 1, 1}, 1.0f};
  auto p2 = IsingSamplingProgram::create(chain, {Block({0, 1, 2, 3})}, {}, dev).unwrap();
  auto s2 = State::create(p2, 1).unwrap();
  s2.set_global({1, 0, 1, 0}).unwrap();
  CHECK(std::fabs(energy(p2, s2).unwrap()[0] - 3.0) < 1e-9);
}

// hinton_init and run_blocks on the 32 x 32 torus (the lattice kernel) equal
// the oracle's chains bit for bit; the f32 block view is the u8 one
void lattice_sweep(Device &dev) {
  std::vector<Block> blocks;
  const IsingEBM ebm = lattice_ebm(32, 0.1, 0.4, 0.05, 1.0f, blocks);
  auto prog = IsingSamplingProgram::create(ebm, blocks, {}, dev).unwrap();
  CHECK(prog.kind() == 0);
  const uint32_t C = 64;
  const auto keys = RngKey(42).split_two();
  auto st = hinton_init(keys.first, prog, C).unwrap();
  auto init = st.get_global().unwrap();
  OracleIsing o(ebm, blocks, {});
  std::vector<uint8_t> want(init.size());
  orc_hinton_init(o.p, keys.first.seed(), C, want.data());
  CHECK(init == want);
  run_blocks(keys.second, prog, st, 10).unwrap();
  uint64_t thr = 0;
  orc_run_blocks(o.p, keys.second.seed(), C, want.data(), 10, 8, &thr);
  const auto got = st.get_global().unwrap();
  CHECK(got == want);
  const auto f = st.get_block(1).unwrap();
  const auto r = prog.block_range(1);
  bool same = true;
  for (uint32_t c = 0; c < C; ++c)
    for (uint64_t i = 0; i < r.second; ++i)
      same &= f[c * r.second + i] == (float)got[c * prog.n_total() + r.first + i];
  CHECK(same);
  run_blocks(RngKey(5), prog, st, 0).unwrap();  // n_iters = 0 is the identity
  CHECK(st.get_global().unwrap() == got);
}

// sample_with_observation with a caller's observer: at every observation it
// sees the state sample_states records for the same key and schedule, with a
// carry kept in the callable; a run started from inside it is refused; the
// f32 form of sample_states records the same observations
void observer_callback(Device &dev) {
  std::vector<Block> blocks;
  const IsingEBM ebm = lattice_ebm(32, 0.2, 0.3, 0.1, 1.0f, blocks);
  auto prog = IsingSamplingProgram::create(ebm, blocks, {}, dev).unwrap();
  const uint32_t C = 40;
  auto st0 = hinton_init(RngKey(3), prog, C).unwrap();
  const auto init = st0.get_global().unwrap();
  const SamplingSchedule sched(3, 5, 2);
  auto st1 = State::create(prog, C).unwrap();
  st1.set_global(init).unwrap();
  const auto want = sample_states(RngKey(11), prog, sched, st1).unwrap();
  auto st2 = State::create(prog, C).unwrap();
  st2.set_global(init).unwrap();
  std::vector<uint8_t> seen;
  uint64_t calls = 0, last = 0;
  int nested = THRML_OK;
  const auto r = sample_with_observation(RngKey(11), prog, sched, st2,
                                         [&](uint64_t it, State &s, void *stream) -> int {
                                           const auto g = s.get_global().unwrap();
                                           seen.insert(seen.end(), g.begin(), g.end());
                                           last = it;
                                           ++calls;
                                           if (it == 1) nested = run_blocks(RngKey(1), prog, s, 1).code();
                                           return stream ? 0 : 1;
                                         });
  CHECK(r.is_ok());
  CHECK(calls == 5 && last == 4);
  CHECK(seen == want);
  CHECK(nested == THRML_EINVAL);
  // the same observations in the StateObserver's f32 representation
  st1.set_global(init).unwrap();
  const auto want_f = sample_states_f32(RngKey(11), prog, sched, st1).unwrap();
  CHECK(want_f.size() == want.size());
  bool same_f = want_f.size() == want.size();
  for (size_t i = 0; same_f && i < want.size(); ++i) same_f = want_f[i] == (float)want[i];
  CHECK(same_f);
  // a nonzero return stops the run and is returned
  const auto stop = sample_with_observation(RngKey(11), prog, sched, st2,
                                            [&](uint64_t it, State &, void *) -> int { return it == 2 ? 7 : 0; });
  CHECK(!stop.is_ok() && stop.code() == 7);
  // an exception thrown by the observer stops the run and comes out of the
  // call; the context then runs normally
  bool thrown = false;
  try {
    sample_with_observation(RngKey(11), prog, sched, st2, [&](uint64_t it, State &, void *) -> int {
      if (it == 1) throw std::runtime_error("observer stops here");
      return 0;
    });
  } catch (const std::runtime_error &e) {
    thrown = std::string(e.what()) == "observer stops here";
  }
  CHECK(thrown);
  CHECK(run_blocks(RngKey(1), prog, st2, 1).is_ok());
  // an observer on this context that runs another context's observer keeps
  // its own guard: a run on this context from inside it is still refused
  Device dev_b = Device::create(0).unwrap();
  auto prog_b = IsingSamplingProgram::create(ebm, blocks, {}, dev_b).unwrap();
  auto st_b = State::create(prog_b, 8).unwrap();
  int inner_calls = 0, after_inner = THRML_OK;
  const auto outer = sample_with_observation(RngKey(11), prog, sched, st2, [&](uint64_t it, State &s, void *) -> int {
    if (it != 0) return 0;
    const auto inner = sample_with_observation(RngKey(2), prog_b, SamplingSchedule(0, 2, 1), st_b,
                                               [&](uint64_t, State &, void *) -> int {
                                                 ++inner_calls;
                                                 return 0;
                                               });
    if (!inner.is_ok()) return 5;
    after_inner = run_blocks(RngKey(1), prog, s, 1).code();
    return 0;
  });
  CHECK(outer.is_ok());
  CHECK(inner_calls == 2);
  CHECK(after_inner == THRML_EINVAL);
}

// estimate_moments on a random graph with a clamped block (the CSR kernel),
// 37 chains: exact integer sums equal the oracle's
void csr_moments_with_clamped_block(Device &dev) {
  const uint32_t n = 300;
  std::mt19937_64 rng(9);
  std::vector<uint32_t> perm(n);
  for (uint32_t i = 0; i < n; ++i) perm[i] = i;
  std::shuffle(perm.begin(), perm.end(), rng);
  std::vector<Block> fb{Block({perm.begin(), perm.begin() + 90}), Block({perm.begin() + 90, perm.begin() + 170}),
                        Block({perm.begin() + 170, perm.begin() + 260})};
  std::vector<Block> cb{Block({perm.begin() + 260, perm.end()})};
  IsingEBM ebm;
  ebm.n_nodes = n;
  ebm.edges = random_edges(n, 900, 3);
  ebm.biases = normal(5, n, 0.0, 0.5);
  ebm.weights = normal(6, ebm.edges.size(), 0.0, 0.6);
  ebm.beta = 0.9f;
  auto prog = IsingSamplingProgram::create(ebm, fb, cb, dev).unwrap();
  CHECK(prog.kind() == 1);
  const uint32_t C = 37;
  std::vector<uint8_t> init((size_t)C * prog.n_total());
  for (auto &x : init) x = (uint8_t)(rng() & 1u);
  auto st = State::create(prog, C).unwrap();
  st.set_global(init).unwrap();
  std::vector<uint32_t> nodes(n);
  for (uint32_t i = 0; i < n; ++i) nodes[i] = i;
  const SamplingSchedule sched(2, 20, 2);
  const auto m = estimate_moments(RngKey(77), nodes, ebm.edges, prog, sched, st).unwrap();
  OracleIsing o(ebm, fb, cb);
  std::vector<int64_t> ns(n), es(ebm.edges.size());
  std::vector<uint32_t> pairs;
  for (const Edge &e : ebm.edges) {
    pairs.push_back(e.first);
    pairs.push_back(e.second);
  }
  uint64_t thr = 0;
  orc_estimate_moments(o.p, 77, orc_schedule{2, 20, 2}, C, init.data(), nodes.data(), n, pairs.data(),
                       ebm.edges.size(), ns.data(), es.data(), 8, &thr);
  CHECK(m.node_sums == ns);
  CHECK(m.edge_sums == es);
  CHECK(st.get_global().unwrap() == init);  // the oracle's final state
  CHECK(std::fabs(m.nodes[0] - (double)ns[0] / (C * 20.0)) < 1e-15);
}

// a categorical (Potts) program: five sweeps equal the oracle's
void categorical_sweep(Device &dev) {
  const Lattice L = make_nearest_neighbor_lattice(16, true);
  const uint32_t q = 4, C = 20;
  const auto W = normal(1104, L.edges.size() * q * q, 0.0, 0.5);
  const auto b = normal(1004, (size_t)L.n_nodes * q, 0.0, 0.3);
  auto prog = CategoricalProgram::create(L.n_nodes, q, L.edges, W, b, {L.upper, L.lower}, dev).unwrap();
  std::mt19937_64 rng(4);
  std::vector<uint8_t> init((size_t)C * prog.n_total());
  for (auto &x : init) x = (uint8_t)(rng() % q);
  auto st = State::create(prog, C).unwrap();
  st.set_global(init).unwrap();
  run_blocks(RngKey(9), prog, st, 5).unwrap();
  std::vector<uint32_t> eu, ev, fo{0}, fn;
  for (const Edge &e : L.edges) {
    eu.push_back(e.first);
    ev.push_back(e.second);
  }
  for (const Block *blk : {&L.upper, &L.lower}) {
    fn.insert(fn.end(), blk->nodes.begin(), blk->nodes.end());
    fo.push_back((uint32_t)fn.size());
  }
  char err[256];
  orc_potts *o = orc_potts_create(L.n_nodes, q, L.edges.size(), eu.data(), ev.data(), W.data(), b.data(), 2,
                                  fo.data(), fn.data(), 0, nullptr, nullptr, err, sizeof err);
  uint64_t thr = 0;
  std::vector<uint16_t> ost(init.begin(), init.end());  // the oracle's uint16 states
  orc_potts_run_blocks(o, 9, C, ost.data(), 5, 8, &thr);
  init.assign(ost.begin(), ost.end());
  CHECK(st.get_global().unwrap() == init);
  std::vector<double> want(C);
  orc_potts_energy(o, C, ost.data(), want.data());
  const auto e = energy(prog, st).unwrap();
  for (uint32_t c = 0; c < C; ++c) CHECK(std::fabs(e[c] - want[c]) < 1e-9 * (1.0 + std::fabs(want[c])));
  orc_potts_destroy(o);
}

// a categorical program with 300 categories (two bytes of state per node)
// through the two-byte global accessors: sweeps and energies equal the
// oracle's; the one-byte read is refused
void categorical_wide_sweep(Device &dev) {
  const uint32_t n = 24, q = 300, C = 9;
  std::vector<Edge> edges;
  for (uint32_t i = 0; i < n; ++i) edges.push_back({i, (i + 1) % n});
  const auto W = normal(1105, edges.size() * q * q, 0.0, 0.7);
  const auto b = normal(1005, (size_t)n * q, 0.0, 0.5);
  Block even, odd;
  for (uint32_t i = 0; i < n; ++i) (i % 2 ? odd : even).nodes.push_back(i);
  auto prog = CategoricalProgram::create(n, q, edges, W, b, {even, odd}, dev).unwrap();
  std::mt19937_64 rng(5);
  std::vector<uint16_t> init((size_t)C * prog.n_total());
  for (auto &x : init) x = (uint16_t)(rng() % q);
  auto st = State::create(prog, C).unwrap();
  st.set_global16(init).unwrap();
  CHECK(st.get_global16().unwrap() == init);
  CHECK(!st.get_global().is_ok());
  run_blocks(RngKey(10), prog, st, 4).unwrap();
  std::vector<uint32_t> eu, ev, fo{0}, fn;
  for (const Edge &e : edges) {
    eu.push_back(e.first);
    ev.push_back(e.second);
  }
  for (const Block *blk : {&even, &odd}) {
    fn.insert(fn.end(), blk->nodes.begin(), blk->nodes.end());
    fo.push_back((uint32_t)fn.size());
  }
  char err[256];
  orc_potts *o = orc_potts_create(n, q, edges.size(), eu.data(), ev.data(), W.data(), b.data(), 2,
                                  fo.data(), fn.data(), 0, nullptr, nullptr, err, sizeof err);
  CHECK(o != nullptr);
  uint64_t thr = 0;
  orc_potts_run_blocks(o, 10, C, init.data(), 4, 8, &thr);
  const auto got = st.get_global16().unwrap();
  CHECK(got == init);
  CHECK(*std::max_element(got.begin(), got.end()) > 255);
  std::vector<double> want(C);
  orc_potts_energy(o, C, init.data(), want.data());
  const auto e = energy(prog, st).unwrap();
  for (uint32_t c = 0; c < C; ++c) CHECK(std::fabs(e[c] - want[c]) < 1e-9 * (1.0 + std::fabs(want[c])));
  orc_potts_destroy(o);
}

// a discrete factor program (a three-spin factor, a spin-categorical and a
// categorical pair factor): sweeps and energies equal the oracle's
void discrete_sweep(Device &dev) {
  const uint32_t ns = 60, nc = 40, q = 3, C = 24, m = 50;
  std::vector<uint8_t> kind(ns + nc, 0);
  for (uint32_t i = ns; i < ns + nc; ++i) kind[i] = 1;
  std::mt19937_64 rng(5);
  auto pick = [&](uint32_t lo, uint32_t n) {
    Block b;
    for (uint32_t i = 0; i < m; ++i) b.nodes.push_back(lo + (uint32_t)(rng() % n));
    return b;
  };
  std::vector<DiscreteFactor> fs(4);
  // three distinct spins per row: s, s + 1, s + 2 (mod ns)
  Block a = pick(0, ns), b2, c2;
  for (uint32_t x : a.nodes) {
    b2.nodes.push_back((x + 1) % ns);
    c2.nodes.push_back((x + 2) % ns);
  }
  fs[0].spin_groups = {a, b2, c2};
  fs[0].weights = normal(21, m, 0.0, 0.6);
  fs[1].spin_groups = {pick(0, ns)};
  fs[1].cat_groups = {pick(ns, nc)};
  fs[1].weights = normal(22, (size_t)m * q, 0.0, 0.6);
  fs[1].d1 = q;
  Block x = pick(ns, nc), y;
  for (uint32_t v : x.nodes) y.nodes.push_back(ns + (v - ns + 1) % nc);
  fs[2].cat_groups = {x, y};
  fs[2].weights = normal(23, (size_t)m * q * q, 0.0, 0.6);
  fs[2].d1 = fs[2].d2 = q;
  fs[2].square = true;  // SquareCategoricalEBMFactor: one merged categorical-head group
  Block all;
  for (uint32_t i = 0; i < ns; ++i) all.nodes.push_back(i);
  fs[3].spin_groups = {all};
  fs[3].weights = normal(24, ns, 0.0, 0.4);
  std::vector<Block> blocks(4);
  for (uint32_t i = 0; i < ns + nc; ++i) blocks[(i < ns ? 0u : 2u) + (i % 2)].nodes.push_back(i);
  auto prog = FactorSamplingProgram::create(kind, q, fs, blocks, dev).unwrap();
  CHECK(prog.kind() == 4);
  std::vector<uint8_t> init((size_t)C * prog.n_total());
  for (uint32_t c = 0; c < C; ++c)
    for (size_t k = 0; k < prog.n_total(); ++k)
      init[(size_t)c * prog.n_total() + k] = (uint8_t)(rng() % (k < ns ? 2u : q));
  auto st = State::create(prog, C).unwrap();
  st.set_global(init).unwrap();
  run_blocks(RngKey(13), prog, st, 4).unwrap();
  std::vector<orc_factor> of(fs.size());
  std::vector<std::vector<uint32_t>> fnodes(fs.size());
  for (size_t i = 0; i < fs.size(); ++i) {
    for (const auto *gs : {&fs[i].spin_groups, &fs[i].cat_groups})
      for (const Block &g : *gs) fnodes[i].insert(fnodes[i].end(), g.nodes.begin(), g.nodes.end());
    const uint32_t batch = (uint32_t)(fs[i].spin_groups.empty() ? fs[i].cat_groups[0] : fs[i].spin_groups[0]).len();
    of[i] = orc_factor{(uint32_t)fs[i].spin_groups.size(), (uint32_t)fs[i].cat_groups.size(), batch,
                       fs[i].d1, fs[i].d2, fnodes[i].data(), fs[i].weights.data(),
                       fs[i].square ? 1u : 0u};
  }
  std::vector<uint32_t> fo{0}, fn;
  for (const Block &blk : blocks) {
    fn.insert(fn.end(), blk.nodes.begin(), blk.nodes.end());
    fo.push_back((uint32_t)fn.size());
  }
  char err[256];
  orc_discrete *o = orc_discrete_create(ns + nc, kind.data(), q, (uint32_t)of.size(), of.data(), 4,
                                        fo.data(), fn.data(), 0, nullptr, nullptr, err, sizeof err);
  CHECK(o != nullptr);
  uint64_t thr = 0;
  std::vector<uint16_t> ost(init.begin(), init.end());  // the oracle holds uint16 states
  orc_discrete_run_blocks(o, 13, C, ost.data(), 4, 8, &thr);
  CHECK(st.get_global().unwrap() == std::vector<uint8_t>(ost.begin(), ost.end()));
  std::vector<double> want(C);
  orc_discrete_energy(o, C, ost.data(), want.data());
  const auto e = energy(prog, st).unwrap();
  for (uint32_t c = 0; c < C; ++c) CHECK(std::fabs(e[c] - want[c]) < 1e-9 * (1.0 + std::fabs(want[c])));
  orc_discrete_destroy(o);
}

// a dense (RBM) program: energies after sweeps equal the oracle's Ising
// energy of the same complete bipartite model (f32 weights, held as bf16
// pieces on the device)
void dense_energy(Device &dev) {
  const uint32_t V = 40, H = 70, C = 90;
  const auto W = normal(11, (size_t)V * H, 0.0, 0.2);
  const auto bv = normal(12, V, 0.0, 0.3), bh = normal(13, H, 0.0, 0.3);
  auto prog = RbmProgram::create(V, H, W, bv, bh, 0.8f, dev).unwrap();
  CHECK(prog.kind() == 3);
  auto st = hinton_init(RngKey(3), prog, C).unwrap();
  run_blocks(RngKey(4), prog, st, 3).unwrap();
  const auto g = st.get_global().unwrap();
  IsingEBM ebm;
  ebm.n_nodes = V + H;
  ebm.biases = bv;
  ebm.biases.insert(ebm.biases.end(), bh.begin(), bh.end());
  ebm.beta = 0.8f;
  double scale = 0.0;
  for (uint32_t v = 0; v < V; ++v)
    for (uint32_t h = 0; h < H; ++h) {
      const float w = W[(size_t)v * H + h];
      ebm.edges.push_back({v, V + h});
      ebm.weights.push_back(w);
      scale += std::fabs(w);
    }
  for (float x : ebm.biases) scale += std::fabs(x);
  OracleIsing o(ebm, prog.free_blocks(), {});
  std::vector<double> want(C);
  orc_ising_energy(o.p, C, g.data(), want.data());
  const auto e = energy(prog, st).unwrap();
  for (uint32_t c = 0; c < C; ++c) CHECK(std::fabs(e[c] - want[c]) <= 1e-7 * 0.8 * scale);
}

// the reference's error strings (blockspec.rs:36-54, program.rs:93-99)
void error_behaviour(Device &dev) {
  std::vector<Block> blocks;
  const IsingEBM ebm = lattice_ebm(4, 0.1, 0.3, 0.05, 1.0f, blocks);
  auto r = IsingSamplingProgram::create(ebm, {blocks[0], Block()}, {}, dev);
  CHECK(r.is_err() && r.error().find("empty block") != std::string::npos);
  r = IsingSamplingProgram::create(ebm, {blocks[0], blocks[0]}, {}, dev);
  CHECK(r.is_err() && r.error().find("twice") != std::string::npos);
  r = IsingSamplingProgram::create(ebm, {blocks[0]}, {}, dev);
  CHECK(r.is_err() && r.error().find("global location map") != std::string::npos);
  auto p1 = IsingSamplingProgram::create(ebm, blocks, {}, dev).unwrap();
  auto p2 = IsingSamplingProgram::create(ebm, blocks, {}, dev).unwrap();
  auto st = State::create(p2, 3).unwrap();
  const auto rr = run_blocks(RngKey(1), p1, st, 1);
  CHECK(rr.is_err() && rr.error().find("another program") != std::string::npos);
  bool threw = false;
  try {
    IsingSamplingProgram::create(ebm, {}, {}, dev).unwrap();
  } catch (const Error &e) {
    threw = e.code == THRML_EINVAL;
  }
  CHECK(threw);
}

struct Case {
  const char *name;
  bool gpu;
  std::function<void(Device *)> fn;
};

}  // namespace

int main(int argc, char **argv) {
  const bool cpu_only = argc > 1 && std::strcmp(argv[1], "--cpu-only") == 0;
  const std::vector<Case> cases = {
      {"rng_split", false, [](Device *) { rng_split(); }},
      {"lattice_graph", false, [](Device *) { lattice_graph(); }},
      {"coloring", false, [](Device *) { coloring(); }},
      {"energy_reference_cases", true, [](Device *d) { energy_reference_cases(*d); }},
      {"lattice_sweep", true, [](Device *d) { lattice_sweep(*d); }},
      {"csr_moments_with_clamped_block", true, [](Device *d) { csr_moments_with_clamped_block(*d); }},
      {"categorical_sweep", true, [](Device *d) { categorical_sweep(*d); }},
      {"categorical_wide_sweep", true, [](Device *d) { categorical_wide_sweep(*d); }},
      {"discrete_sweep", true, [](Device *d) { discrete_sweep(*d); }},
      {"dense_energy", true, [](Device *d) { dense_energy(*d); }},
      {"error_behaviour", true, [](Device *d) { error_behaviour(*d); }},
      {"observer_callback", true, [](Device *d) { observer_callback(*d); }},
  };
  std::unique_ptr<Device> dev;
  int failed = 0, run = 0;
  for (const Case &c : cases) {
    if (c.gpu && cpu_only) continue;
    if (c.gpu && !dev) dev.reset(new Device(Device::create(0).unwrap()));
    std::printf("[case] %s\n", c.name);
    std::fflush(stdout);
    g_fail = 0;
    try {
      c.fn(dev.get());
    } catch (const std::exception &e) {
      std::printf("  exception: %s\n", e.what());
      ++g_fail;
    }
    std::printf("%s %s\n", g_fail ? "FAIL" : "PASS", c.name);
    failed += g_fail ? 1 : 0;
    ++run;
  }
  std::printf("%d of %d cases passed\n", run - failed, run);
  return failed ? 1 : 0;
}
