// capi.hip -- the C ABI of libthrml_hip.so: contexts, program construction,
// states and the sweep drivers.  See include/thrml_hip.h for the contract.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <numeric>
#include <string>
#include <vector>

#include "dev_util.hpp"
#include "internal.hpp"
#include "thrml_math.hpp"
#include "thrml_rng.hpp"

namespace thrml {

static thread_local std::string g_last_error;

void set_error(const std::string &msg) { g_last_error = msg; }
int fail(int code, const std::string &msg) {
  g_last_error = msg;
  return code;
}
int hip_fail(hipError_t e, const char *what) {
  g_last_error = std::string("HIP error in ") + what + ": " + hipGetErrorString(e);
  return THRML_EHIP;
}

}  // namespace thrml

using namespace thrml;

// ---------------------------------------------------------------------------
// Key store of thrml_run_blocks_noalloc: a fixed device array in place of
// the context's growable key buffer.  Every GPU the library runs on holds its
// own copy until the process ends.  In host code the array's name is only a
// host-side stand-in: kernels and copies get the device address that
// hipGetSymbolAddress returns with that device current, kept per device.
static __device__ __align__(256) uint32_t scratch[THRML_NOALLOC_KEY_BYTES / sizeof(uint32_t)];

namespace {
constexpr int kMaxDevices = 64;  // device ordinals the per-device tables hold
struct ScratchSlot {
  bool done = false;
  hipError_t err = hipSuccess;
  uint32_t *ptr = nullptr;
  // Calls from different streams (contexts) on one GPU share the array: each
  // call records done_ev on its stream after its last launch, and a call on
  // another stream first makes its stream wait for that event.
  hipEvent_t done_ev = nullptr;
  hipStream_t last = nullptr;  // stream of the latest call (under use_mu)
};
std::mutex g_scratch_mu;
ScratchSlot g_scratch[kMaxDevices];
std::mutex g_scratch_use_mu[kMaxDevices];  // held across one call's launches

// Resolves the array's address on `device` and creates its event, once per
// device; the caller has made `device` current.  A failure is kept for the
// error message and set-up is tried again at the next context creation.
void scratch_setup(int device) {
  if (device < 0 || device >= kMaxDevices) return;
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  ScratchSlot &s = g_scratch[device];
  if (s.done) return;
  void *ptr = nullptr;
  s.err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (s.err != hipSuccess) return;
  if (!s.done_ev) {
    s.err = hipEventCreateWithFlags(&s.done_ev, hipEventDisableTiming);
    if (s.err != hipSuccess) {
      s.done_ev = nullptr;
      return;
    }
  }
  s.ptr = static_cast<uint32_t *>(ptr);
  s.done = true;
}

ScratchSlot scratch_slot(int device) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  return (device >= 0 && device < kMaxDevices) ? g_scratch[device] : ScratchSlot{};
}

// The hardware-math self-check behind the sweep kernels' exact fast paths,
// run once per device at the first program creation and kept: programs are
// refused on a device whose measured errors exceed what the fast paths
// assume (the Gumbel margin and the spin decision band).
struct FastMathSlot {
  bool done = false;
  bool ok = false;
  float v[3] = {0.f, 0.f, 0.f};
};
std::mutex g_fm_mu;
FastMathSlot g_fm[kMaxDevices];
}  // namespace

// The bounds the kernels' fast paths assume of the measured errors:
// Gumbel |fast - exact| <= GUMBEL_FAST_ERR, and the relative errors of the
// hardware e^(-2g) and of the exact sigmoid plus one rounding below the
// spin band.
extern "C" int thrml_fast_math_bounds_ok(const float *v) {
  if (!v) return 0;
  return v[0] <= GUMBEL_FAST_ERR && (double)v[1] + (double)v[2] + 0x1p-23 < (double)SPIN_BAND;
}

namespace thrml {
// Runs (once per device) and consults the cached self-check.
int fast_math_gate(thrml_ctx *ctx, float *v_out, int *ok_out) {
  const int dev = ctx->device;
  if (dev < 0 || dev >= kMaxDevices)
    return fail(THRML_EUNSUPPORTED, "device ordinal " + std::to_string(dev) +
                                        " is above the 64 the library's per-device tables hold");
  std::lock_guard<std::mutex> lk(g_fm_mu);
  FastMathSlot &s = g_fm[dev];
  if (!s.done) {
    float v[3];
    if (int rc = launch_fast_math_check(ctx, v)) return rc;  // not cached: tried again
    std::memcpy(s.v, v, sizeof v);
    s.ok = thrml_fast_math_bounds_ok(v) != 0;
    s.done = true;
  }
  if (v_out) std::memcpy(v_out, s.v, sizeof s.v);
  if (ok_out) *ok_out = s.ok ? 1 : 0;
  if (!s.ok && !ok_out)
    return fail(THRML_EUNSUPPORTED,
                "the hardware exp/log of device " + std::to_string(dev) +
                    " exceed the error bounds the sweep kernels' exact decisions rely on "
                    "(thrml_fast_math_check: gumbel " + std::to_string(s.v[0]) + ", exp " +
                    std::to_string(s.v[1]) + ", sigmoid " + std::to_string(s.v[2]) + ")");
  return THRML_OK;
}
}  // namespace thrml

int thrml_ctx::time_begin(int k, hipEvent_t *start) {
  *start = nullptr;
  if (!timing) return 0;
  if (timing == 2 && slots[k].span0) return 0;
  hipEvent_t a;
  if (hipEventCreate(&a) != hipSuccess) return 1;
  if (hipEventRecord(a, stream) != hipSuccess) return 1;
  if (timing == 2)
    slots[k].span0 = a;
  else
    *start = a;
  return 0;
}

int thrml_ctx::time_end(int k, hipEvent_t start) {
  if (timing == 2) {
    slots[k].span_n += 1;
    return THRML_OK;
  }
  if (!timing || !start) return THRML_OK;
  hipEvent_t b;
  THRML_HIP(hipEventCreate(&b));
  THRML_HIP(hipEventRecord(b, stream));
  slots[k].ev.push_back(start);
  slots[k].ev.push_back(b);
  if (slots[k].ev.size() >= 4096) return flush_timing(k);
  return THRML_OK;
}

int thrml_ctx::flush_timing(int k) {
  auto &v = slots[k].ev;
  if (slots[k].span0) {
    // span mode: the stream time from before the first launch to now (the
    // end of the last one, and of any work queued after it), over the count
    hipEvent_t b;
    THRML_HIP(hipEventCreate(&b));
    THRML_HIP(hipEventRecord(b, stream));
    THRML_HIP(hipEventSynchronize(b));
    float ms = 0.f;
    THRML_HIP(hipEventElapsedTime(&ms, slots[k].span0, b));
    acc_ms[k] += ms;
    acc_n[k] += slots[k].span_n;
    (void)hipEventDestroy(slots[k].span0);
    (void)hipEventDestroy(b);
    slots[k].span0 = nullptr;
    slots[k].span_n = 0;
  }
  if (v.empty()) return THRML_OK;
  THRML_HIP(hipEventSynchronize(v.back()));
  for (size_t i = 0; i + 1 < v.size(); i += 2) {
    float ms = 0.f;
    THRML_HIP(hipEventElapsedTime(&ms, v[i], v[i + 1]));
    acc_ms[k] += ms;
    acc_n[k] += 1;
  }
  for (auto e : v) (void)hipEventDestroy(e);
  v.clear();
  return THRML_OK;
}

extern "C" int thrml_version(void) { return 100; }
extern "C" const char *thrml_last_error(void) { return g_last_error.c_str(); }

extern "C" int thrml_ctx_create(int device_ordinal, thrml_ctx **out) {
  if (!out) return fail(THRML_EINVAL, "out is NULL");
  int n = 0;
  THRML_HIP(hipGetDeviceCount(&n));
  if (device_ordinal < 0 || device_ordinal >= n)
    return fail(THRML_EINVAL, "device ordinal " + std::to_string(device_ordinal) + " out of range (" +
                                  std::to_string(n) + " devices)");
  THRML_HIP(hipSetDevice(device_ordinal));
  scratch_setup(device_ordinal);  // thrml_run_blocks_noalloc's key array
  auto *c = new thrml_ctx();
  c->device = device_ordinal;
  hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete c;
    return hip_fail(e, "hipStreamCreateWithFlags");
  }
  c->own_stream = true;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device_ordinal) == hipSuccess) c->cu_count = prop.multiProcessorCount;
  *out = c;
  return THRML_OK;
}

extern "C" void thrml_ctx_destroy(thrml_ctx *ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  for (int k = 0; k < 2; ++k) {
    for (auto e : ctx->slots[k].ev) (void)hipEventDestroy(e);
    if (ctx->slots[k].span0) (void)hipEventDestroy(ctx->slots[k].span0);
  }
  if (ctx->own_stream) (void)hipStreamDestroy(ctx->stream);
  delete ctx;
}

extern "C" int thrml_ctx_set_stream(thrml_ctx *ctx, void *s) {
  if (!ctx) return fail(THRML_EINVAL, "ctx is NULL");
  if (ctx->own_stream) {
    THRML_HIP(hipStreamSynchronize(ctx->stream));
    THRML_HIP(hipStreamDestroy(ctx->stream));
  }
  ctx->stream = reinterpret_cast<hipStream_t>(s);
  ctx->own_stream = false;
  return THRML_OK;
}

extern "C" void *thrml_ctx_get_stream(thrml_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

extern "C" int thrml_ctx_synchronize(thrml_ctx *ctx) {
  if (!ctx) return fail(THRML_EINVAL, "ctx is NULL");
  THRML_HIP(hipStreamSynchronize(ctx->stream));
  return THRML_OK;
}

extern "C" int thrml_ctx_enable_timing(thrml_ctx *ctx, int enable) {
  if (!ctx) return fail(THRML_EINVAL, "ctx is NULL");
  if (enable < 0 || enable > 2) return fail(THRML_EINVAL, "timing mode must be 0, 1 or 2");
  for (int k = 0; k < 2; ++k) {
    if (int rc = ctx->flush_timing(k)) return rc;
    ctx->acc_ms[k] = 0;
    ctx->acc_n[k] = 0;
  }
  ctx->timing = enable;
  return THRML_OK;
}

extern "C" int thrml_ctx_kernel_time(thrml_ctx *ctx, int kernel, double *avg_ms, uint64_t *count) {
  if (!ctx || kernel < 0 || kernel > 1) return fail(THRML_EINVAL, "bad ctx or kernel index");
  if (int rc = ctx->flush_timing(kernel)) return rc;
  if (count) *count = ctx->acc_n[kernel];
  if (avg_ms) *avg_ms = ctx->acc_n[kernel] ? ctx->acc_ms[kernel] / (double)ctx->acc_n[kernel] : 0.0;
  return THRML_OK;
}

// ---------------------------------------------------------------------------
// RngKey
extern "C" int thrml_rng_split(uint64_t key, uint64_t n, uint64_t *out) {
  if (n && !out) return fail(THRML_EINVAL, "out is NULL");
  if (n == 1) {
    out[0] = key;
    return THRML_OK;
  }
  if (n == 0) return THRML_OK;
  const Key8 k = seed_from_u64(key);
  uint32_t blk[16];
  for (uint64_t i = 0; i < n; ++i) {
    if ((i & 7u) == 0) chacha_block<8>(k.k, i >> 3, blk);
    const uint32_t j = (uint32_t)(i & 7u) * 2u;
    out[i] = (uint64_t)blk[j] | ((uint64_t)blk[j + 1] << 32);
  }
  return THRML_OK;
}

// ---------------------------------------------------------------------------
// graph builders
extern "C" int64_t thrml_lattice_edges(uint32_t side, int torus, uint32_t *u, uint32_t *v) {
  if (side == 0) return fail(THRML_EINVAL, "side_len must be positive");
  const uint64_t L = (side + 1u) / 2u * 2u;
  int64_t ne = 0;
  // canonical order: idx ascending, jump (1,0) then (0,1), edge (min, max);
  // a repeat can only occur on the 2x2 torus.
  std::vector<uint64_t> seen;
  for (uint64_t idx = 0; idx < L * L; ++idx) {
    const uint64_t i = idx / L, j = idx % L;
    for (int t = 0; t < 2; ++t) {
      uint64_t ii = i + (t == 0), jj = j + (t == 1);
      if (torus) {
        ii %= L;
        jj %= L;
      } else if (ii >= L || jj >= L) {
        continue;
      }
      const uint64_t tgt = ii * L + jj;
      const uint64_t a = std::min(idx, tgt), b = std::max(idx, tgt);
      if (a == b) continue;
      if (L <= 2) {
        const uint64_t key = a * L * L + b;
        if (std::find(seen.begin(), seen.end(), key) != seen.end()) continue;
        seen.push_back(key);
      }
      if (u && v) {
        u[ne] = (uint32_t)a;
        v[ne] = (uint32_t)b;
      }
      ++ne;
    }
  }
  return ne;
}

extern "C" int thrml_lattice_blocks(uint32_t side, uint32_t *upper, uint32_t *lower) {
  if (side == 0) return fail(THRML_EINVAL, "side_len must be positive");
  const uint32_t L = (side + 1u) / 2u * 2u;
  uint64_t a = 0, b = 0;
  for (uint32_t idx = 0; idx < L * L; ++idx) {
    if ((((idx / L) + (idx % L)) & 1u) == 0)
      upper[a++] = idx;
    else
      lower[b++] = idx;
  }
  return THRML_OK;
}

extern "C" int64_t thrml_greedy_coloring(uint32_t n, uint64_t ne, const uint32_t *u,
                                         const uint32_t *v, uint32_t *color) {
  std::vector<uint64_t> off((size_t)n + 1, 0);
  for (uint64_t e = 0; e < ne; ++e) {
    if (u[e] >= n || v[e] >= n) return fail(THRML_EINVAL, "edge endpoint out of range");
    off[u[e] + 1]++;
    off[v[e] + 1]++;
  }
  for (uint32_t i = 0; i < n; ++i) off[i + 1] += off[i];
  std::vector<uint32_t> adj(off[n]);
  std::vector<uint64_t> fill(off.begin(), off.end() - 1);
  for (uint64_t e = 0; e < ne; ++e) {
    adj[fill[u[e]]++] = v[e];
    adj[fill[v[e]]++] = u[e];
  }
  const uint32_t none = 0xffffffffu;
  std::fill(color, color + n, none);
  std::vector<uint8_t> used;
  uint32_t ncol = 0;
  for (uint32_t x = 0; x < n; ++x) {
    const uint64_t deg = off[x + 1] - off[x];
    used.assign(deg + 2, 0);
    for (uint64_t k = off[x]; k < off[x + 1]; ++k) {
      const uint32_t c = color[adj[k]];
      if (c != none && c <= deg) used[c] = 1;
    }
    uint32_t c = 0;
    while (used[c]) ++c;
    color[x] = c;
    ncol = std::max(ncol, c + 1);
  }
  return ncol;
}

namespace {
// u32 keystream reader of ChaCha8Rng::seed_from_u64(seed)
struct WordStream {
  Key8 k;
  uint64_t w = 0;
  uint32_t blk[16];
  explicit WordStream(uint64_t seed) : k(seed_from_u64(seed)) {}
  uint32_t next() {
    if ((w & 15u) == 0) chacha_block<8>(k.k, w >> 4, blk);
    return blk[(w++) & 15u];
  }
  double unit() { return ((double)next() + 0.5) / 4294967296.0; }
};
}  // namespace

extern "C" int64_t thrml_erdos_renyi(uint32_t n, double p, uint64_t seed, uint32_t *u,
                                     uint32_t *v, uint64_t cap) {
  if (!(p > 0.0 && p < 1.0)) return fail(THRML_EINVAL, "p must lie in (0, 1)");
  // Geometric skipping over the pairs (w < v) in (v, w) order
  // (Batagelj & Brandes 2005), then ascending (min, max) order.
  WordStream rs(seed);
  const double lq = std::log(1.0 - p);
  std::vector<uint64_t> e;
  int64_t vv = 1, w = -1;
  while (vv < (int64_t)n) {
    const double r = rs.unit();
    w = w + 1 + (int64_t)std::floor(std::log(1.0 - r) / lq);
    while (w >= vv && vv < (int64_t)n) {
      w -= vv;
      vv += 1;
    }
    if (vv < (int64_t)n) e.push_back(((uint64_t)w << 32) | (uint64_t)vv);
  }
  if (e.size() > cap || !u || !v) return (int64_t)e.size();
  std::sort(e.begin(), e.end());
  for (size_t i = 0; i < e.size(); ++i) {
    u[i] = (uint32_t)(e[i] >> 32);
    v[i] = (uint32_t)(e[i] & 0xffffffffu);
  }
  return (int64_t)e.size();
}

namespace {
// rand 0.8.5 StdRng (rand_chacha 0.3.1 ChaCha12Rng) from seed_from_u64:
// next_u32 reads the ChaCha12 keystream word by word, blocks in counter order.
struct StdRng32 {
  Key8 k;
  uint64_t w = 0;
  uint32_t blk[16];
  explicit StdRng32(uint64_t seed) : k(seed_from_u64(seed)) {}
  uint32_t next_u32() {
    if ((w & 15u) == 0) chacha_block<12>(k.k, w >> 4, blk);
    return blk[(w++) & 15u];
  }
  // gen_range(0..n) for u32 (rand 0.8.5 UniformInt::sample_single): widening
  // multiply by the range, rejecting low halves above the zone
  // (range << leading_zeros(range)) - 1.
  uint32_t below(uint32_t n) {
    const uint32_t zone = (n << __builtin_clz(n)) - 1u;
    for (;;) {
      const uint64_t m = (uint64_t)next_u32() * n;
      if ((uint32_t)m <= zone) return (uint32_t)(m >> 32);
    }
  }
};
}  // namespace

// get_double_grid (crates/thrml-models/tests/test_train_mnist.rs:37-115).
extern "C" int64_t thrml_double_grid(uint32_t side, const uint32_t *jumps, uint32_t n_jumps,
                                     uint32_t n_visible, uint64_t seed, uint32_t *u, uint32_t *v,
                                     uint32_t *visible) {
  const uint64_t size = (uint64_t)side * side;
  if (side == 0 || size >= 0x7fffffffull) return fail(THRML_EINVAL, "side_len out of range");
  if (n_visible > size) return fail(THRML_EINVAL, "n_visible must be <= grid size");
  if (n_jumps && !jumps) return fail(THRML_EINVAL, "jumps is NULL");
  const int64_t ne = (int64_t)size * (1 + 4 * (int64_t)n_jumps);
  if (!u || !v || !visible) return ne;
  // edges (upper i, lower j) as node ids (i, size + j): first i -> i, then per
  // jump d the four torus neighbours at distance d in the order -row, +row,
  // -col, +col
  const int64_t L = side;
  auto idx = [&](int64_t i, int64_t j) {
    i = ((i % L) + L) % L;
    j = ((j % L) + L) % L;
    return (uint32_t)(i * L + j);
  };
  int64_t e = 0;
  for (uint64_t x = 0; x < size; ++x, ++e) {
    u[e] = (uint32_t)x;
    v[e] = (uint32_t)(size + x);
  }
  for (uint32_t q = 0; q < n_jumps; ++q) {
    const int64_t d = jumps[q];
    for (uint64_t x = 0; x < size; ++x) {
      const int64_t i = (int64_t)x / L, j = (int64_t)x % L;
      const uint32_t t[4] = {idx(i - d, j), idx(i + d, j), idx(i, j - d), idx(i, j + d)};
      for (int k = 0; k < 4; ++k, ++e) {
        u[e] = (uint32_t)x;
        v[e] = (uint32_t)(size + t[k]);
      }
    }
  }
  // visible nodes: the first n_visible of 0..size shuffled by SliceRandom::
  // shuffle (rand 0.8.5: for i from len-1 down to 1, swap i with gen_range(0..i+1))
  std::vector<uint32_t> perm(size);
  for (uint64_t x = 0; x < size; ++x) perm[x] = (uint32_t)x;
  StdRng32 rng(seed);
  for (uint64_t i = size - 1; i >= 1; --i) std::swap(perm[i], perm[rng.below((uint32_t)i + 1u)]);
  std::copy(perm.begin(), perm.begin() + n_visible, visible);
  return ne;
}

extern "C" int thrml_param_normal(uint64_t seed, uint64_t n, double mean, double std_, float *out) {
  WordStream rs(seed);
  const double two_pi = 6.283185307179586476925286766559;
  for (uint64_t i = 0; i < n; i += 2) {
    const double u0 = rs.unit(), u1 = rs.unit();
    const double r = std::sqrt(-2.0 * std::log(u0));
    out[i] = (float)(mean + std_ * r * std::cos(two_pi * u1));
    if (i + 1 < n) out[i + 1] = (float)(mean + std_ * r * std::sin(two_pi * u1));
  }
  return THRML_OK;
}

// ---------------------------------------------------------------------------
// program construction helpers
namespace {

int build_blocks(thrml_prog *p, uint32_t n_nodes, uint32_t n_free, const uint32_t *foff,
                 const uint32_t *fnodes, uint32_t n_clamp, const uint32_t *coff,
                 const uint32_t *cnodes) {
  if ((n_free && (!foff || !fnodes)) || (n_clamp && (!coff || !cnodes)))
    return fail(THRML_EINVAL, "block arrays are NULL");
  p->n_free = n_free;
  p->n_clamped = n_clamp;
  const uint32_t nb = n_free + n_clamp;
  p->blk_off.assign((size_t)nb + 1, 0);
  for (uint32_t b = 0; b < nb; ++b) {
    const uint64_t len = b < n_free ? (uint64_t)foff[b + 1] - foff[b]
                                    : (uint64_t)coff[b - n_free + 1] - coff[b - n_free];
    if (len == 0) return fail(THRML_EINVAL, "Encountered an empty block in BlockSpec");
    p->blk_off[b + 1] = p->blk_off[b] + len;
  }
  p->n_total = p->blk_off[nb];
  if (p->n_total >= 0xffffffffull) return fail(THRML_EUNSUPPORTED, "more than 2^32-1 block nodes");
  p->node_pos.assign(n_nodes, -1);
  p->pos_node.assign(p->n_total, 0);
  for (uint32_t b = 0; b < nb; ++b) {
    for (uint64_t k = p->blk_off[b]; k < p->blk_off[b + 1]; ++k) {
      const uint32_t node = b < n_free ? fnodes[foff[b] + (k - p->blk_off[b])]
                                       : cnodes[coff[b - n_free] + (k - p->blk_off[b])];
      if (node >= n_nodes) return fail(THRML_EINVAL, "Node not found in global location map");
      if (p->node_pos[node] >= 0) return fail(THRML_EINVAL, "Node appears twice in blocks");
      p->node_pos[node] = (int64_t)k;
      p->pos_node[k] = node;
    }
  }
  return THRML_OK;
}

// A program table: uploaded and counted in the program's device bytes.
template <class T>
int upload(thrml_prog *p, DevBuf &buf, const std::vector<T> &v) {
  if (int rc = upload_to(p->ctx, buf, v)) return rc;
  p->device_bytes += buf.bytes;
  return THRML_OK;
}

// Does the program match the 2-colour checkerboard of an L x L lattice with
// every slot pointing at one of the 4 lattice neighbours?  If so fill dir.
bool detect_lattice(thrml_prog *p, uint32_t n_nodes, const std::vector<uint32_t> &row_off,
                    const std::vector<uint32_t> &slot_pos, std::vector<uint32_t> &dir) {
  if (p->n_free != 2 || p->n_clamped != 0) return false;
  const uint32_t L = (uint32_t)std::llround(std::sqrt((double)n_nodes));
  if ((uint64_t)L * L != n_nodes || L < 32 || (L % 32u) != 0u) return false;
  const uint32_t half = L / 2;
  if (p->blk_off[1] != (uint64_t)n_nodes / 2 || p->n_total != n_nodes) return false;
  uint32_t par[2];
  for (uint32_t b = 0; b < 2; ++b) {
    const uint32_t first = p->pos_node[p->blk_off[b]];
    if (first > 1) return false;
    par[b] = first;
  }
  if (par[0] == par[1]) return false;
  for (uint32_t b = 0; b < 2; ++b) {
    for (uint64_t k = p->blk_off[b]; k < p->blk_off[b + 1]; ++k) {
      const uint64_t i = k - p->blk_off[b];
      const uint64_t r = i / half, t = i % half;
      const uint64_t j = 2 * t + ((r + par[b]) & 1u);
      if (p->pos_node[k] != r * L + j) return false;
    }
  }
  dir.assign(slot_pos.size(), 0);
  for (uint64_t k = 0; k < p->n_total; ++k) {
    const uint32_t node = p->pos_node[k];
    const uint32_t r = node / L, j = node % L;
    const uint32_t nb[4] = {r * L + (j + L - 1) % L, r * L + (j + 1) % L, ((r + L - 1) % L) * L + j,
                            ((r + 1) % L) * L + j};
    const uint32_t b = k < p->blk_off[1] ? 0u : 1u;
    for (uint32_t s = row_off[k]; s < row_off[k + 1]; ++s) {
      const uint32_t tp = slot_pos[s];
      const uint32_t tb = tp < p->blk_off[1] ? 0u : 1u;
      if (tb == b) return false;
      const uint32_t tn = p->pos_node[tp];
      int d = -1;
      for (int q = 0; q < 4; ++q)
        if (nb[q] == tn) {
          d = q;
          break;
        }
      if (d < 0) return false;
      dir[s] = (uint32_t)d;
    }
  }
  p->L = L;
  p->half = half;
  p->parity[0] = par[0];
  p->parity[1] = par[1];
  return true;
}

// An RBM-shaped model for the matrix-core path, taken only when the caller
// sets THRML_ISING_DENSE: two blocks (free ++ clamped) of at least
// THRML_DENSE_MIN_SIDE nodes whose edges are exactly the complete bipartite
// graph between them, each pair once in either orientation.  Fills the spec
// with side s = block s: W[i][j] couples block 0's i-th node with block 1's
// j-th.  Whether every weight is a sum of at most three normal bf16 values
// (every finite f32 of magnitude above about 2^-110) is found on the device
// by dense_program_create, which refuses the program otherwise.
bool dense_candidate(const thrml_ising_desc *d, const thrml_prog *p, DenseSpec &s) {
  if (!(d->flags & THRML_ISING_DENSE)) return false;
  if (p->n_free + p->n_clamped != 2) return false;
  const uint64_t n0 = p->blk_off[1], n1 = p->blk_off[2] - p->blk_off[1];
  if (n0 < THRML_DENSE_MIN_SIDE || n1 < THRML_DENSE_MIN_SIDE || d->n_edges != n0 * n1) return false;
  std::vector<float> w(n0 * n1);
  std::vector<uint8_t> seen(n0 * n1, 0);
  for (uint64_t e = 0; e < d->n_edges; ++e) {
    if (d->edge_u[e] >= d->n_nodes || d->edge_v[e] >= d->n_nodes) return false;
    const int64_t pa = p->node_pos[d->edge_u[e]], pb = p->node_pos[d->edge_v[e]];
    if (pa < 0 || pb < 0 || ((uint64_t)pa < n0) == ((uint64_t)pb < n0)) return false;
    const uint64_t i = (uint64_t)std::min(pa, pb), j = (uint64_t)std::max(pa, pb) - n0;
    if (seen[i * n1 + j]) return false;
    seen[i * n1 + j] = 1;
    w[i * n1 + j] = d->weights[e];
  }
  s.n_nodes = d->n_nodes;
  s.side_nodes[0].assign(p->pos_node.begin(), p->pos_node.begin() + (long)n0);
  s.side_nodes[1].assign(p->pos_node.begin() + (long)n0, p->pos_node.end());
  s.w = std::move(w);
  s.bias.assign(d->biases, d->biases + d->n_nodes);
  s.beta = d->beta;
  s.block_side[0] = 0;
  s.block_side[1] = 1;
  s.n_free = p->n_free;
  return true;
}

}  // namespace

namespace thrml {

int set_superblocks(thrml_prog *p, uint32_t n_sb, const uint32_t *offsets) {
  const uint32_t nf = p->n_free;
  if (n_sb == 0) {
    p->sb_off.resize((size_t)nf + 1);
    for (uint32_t b = 0; b <= nf; ++b) p->sb_off[b] = b;
  } else {
    if (!offsets) return fail(THRML_EINVAL, "superblock_offsets is NULL");
    if (offsets[0] != 0 || offsets[n_sb] != nf)
      return fail(THRML_EINVAL, "superblock offsets must start at 0 and end at the number of free blocks");
    for (uint32_t s = 0; s < n_sb; ++s)
      if (offsets[s + 1] < offsets[s])
        return fail(THRML_EINVAL, "superblock offsets must not decrease");
    p->sb_off.assign(offsets, offsets + n_sb + 1);
  }
  p->blk_sb.assign(nf, 0);
  for (uint32_t s = 0; s + 1 < p->sb_off.size(); ++s)
    for (uint32_t b = p->sb_off[s]; b < p->sb_off[s + 1]; ++b) p->blk_sb[b] = s;
  p->staged.assign(nf, 0);
  p->stage_width.assign(p->sb_off.size() - 1, 0);
  p->stage_max = 0;
  return THRML_OK;
}

void plan_staging(thrml_prog *p) {
  p->stage_max = 0;
  for (uint32_t s = 0; s + 1 < p->sb_off.size(); ++s) {
    const uint32_t first = p->sb_off[s], end = p->sb_off[s + 1];
    if (first == end) continue;
    // the last block of a superblock runs after every other block of it has
    // read the state, so it writes in place unless it reads its own block
    const uint32_t stage_end = p->intra_block_edges ? end : end - 1;
    for (uint32_t b = first; b < stage_end; ++b) p->staged[b] = 1;
    if (stage_end > first) {
      p->stage_width[s] = p->blk_off[stage_end] - p->blk_off[first];
      p->stage_max = std::max(p->stage_max, p->stage_width[s]);
    }
  }
}

int commit_superblock(thrml_prog *p, thrml_state *st, uint32_t s) {
  const uint64_t width = p->stage_width[s];
  if (!width) return THRML_OK;
  const uint64_t at = p->blk_off[p->sb_off[s]];
  hipStream_t stream = p->ctx->stream;
  if (byte_layout(p)) {
    THRML_HIP(hipMemcpyAsync(st->cat.as<uint8_t>() + at * st->Cp * p->cat_bytes, st->scratch.p,
                             width * st->Cp * p->cat_bytes, hipMemcpyDeviceToDevice, stream));
  } else {
    THRML_HIP(hipMemcpy2DAsync(st->words.as<uint64_t>() + at, p->n_total * 8, st->scratch.p,
                               width * 8, width * 8, (size_t)st->G * p->planes,
                               hipMemcpyDeviceToDevice, stream));
  }
  return THRML_OK;
}

}  // namespace thrml

extern "C" int thrml_ising_program_create(thrml_ctx *ctx, const thrml_ising_desc *d,
                                          thrml_prog **out) {
  if (!ctx || !d || !out) return fail(THRML_EINVAL, "NULL argument");
  if (d->n_free_blocks == 0) return fail(THRML_EINVAL, "Number of samplers (0) must match number of free blocks (0)");
  if (d->n_edges && (!d->edge_u || !d->edge_v || !d->weights))
    return fail(THRML_EINVAL, "edge arrays are NULL");
  if (d->n_nodes && !d->biases) return fail(THRML_EINVAL, "biases is NULL");
  if (d->flags & ~THRML_ISING_DENSE) return fail(THRML_EINVAL, "unknown flags");
  // slot offsets are 32-bit: every edge takes one slot at each endpoint
  if (d->n_edges > 0x7fffffffull) return fail(THRML_EUNSUPPORTED, "more than 2^31-1 edges");
  THRML_HIP(hipSetDevice(ctx->device));
  if (int rc = fast_math_gate(ctx, nullptr, nullptr)) return rc;
  auto *p = new thrml_prog();
  p->ctx = ctx;
  int rc = build_blocks(p, d->n_nodes, d->n_free_blocks, d->free_offsets, d->free_nodes,
                        d->n_clamped_blocks, d->clamped_offsets, d->clamped_nodes);
  if (!rc) rc = set_superblocks(p, d->n_superblocks, d->superblock_offsets);
  if (rc) {
    delete p;
    return rc;
  }
  const bool one_per_block = p->sb_off.size() == (size_t)p->n_free + 1 &&
                             std::equal(p->sb_off.begin() + 1, p->sb_off.end(), p->sb_off.begin(),
                                        [](uint32_t a, uint32_t b) { return a == b + 1; });
  if (one_per_block) {
    DenseSpec ds;
    if (dense_candidate(d, p, ds)) {
      thrml_prog *dp = nullptr;
      const int drc = dense_program_create(ctx, ds, &dp);
      if (drc == THRML_OK) {
        delete p;
        *out = dp;
        return THRML_OK;
      }
      if (drc != THRML_EUNSUPPORTED) {
        delete p;
        return drc;
      }
      // a weight with no exact bf16-piece form: the CSR kernel takes the model
    }
  }
  p->beta = d->beta;
  p->bias_raw.assign(d->biases, d->biases + d->n_nodes);
  p->eu.assign(d->edge_u, d->edge_u + d->n_edges);
  p->ev.assign(d->edge_v, d->edge_v + d->n_edges);
  p->w_raw.assign(d->weights, d->weights + d->n_edges);

  // Slots of every free position in the reference's order
  // (crates/thrml-samplers/src/program.rs:102-200 over the edge group of
  // crates/thrml-models/src/discrete_ebm.rs:390-453): u-role edges ascending,
  // then v-role edges ascending; weight fl(beta * J).
  const uint64_t nf = p->blk_off[p->n_free];
  std::vector<uint32_t> row_off(nf + 1, 0);
  for (uint64_t e = 0; e < d->n_edges; ++e) {
    const uint32_t a = d->edge_u[e], b = d->edge_v[e];
    if (a >= d->n_nodes || b >= d->n_nodes) {
      delete p;
      return fail(THRML_EINVAL, "Node not found in global location map");
    }
    const int64_t pa = p->node_pos[a], pb = p->node_pos[b];
    if (pa >= 0 && (uint64_t)pa < nf) row_off[pa + 1]++;
    if (pb >= 0 && (uint64_t)pb < nf) row_off[pb + 1]++;
  }
  for (uint64_t k = 0; k < nf; ++k) row_off[k + 1] += row_off[k];
  const uint64_t ns = row_off[nf];
  std::vector<uint32_t> slot_pos(ns);
  std::vector<float> slot_w(ns);
  std::vector<uint32_t> fill(row_off.begin(), row_off.end() - 1);
  bool intra = false;
  auto blk_of = [&](uint64_t pos) {
    return (uint32_t)(std::upper_bound(p->blk_off.begin(), p->blk_off.end(), pos) - p->blk_off.begin() - 1);
  };
  for (int pass = 0; pass < 2; ++pass) {
    for (uint64_t e = 0; e < d->n_edges; ++e) {
      const uint32_t head = pass == 0 ? d->edge_u[e] : d->edge_v[e];
      const uint32_t tail = pass == 0 ? d->edge_v[e] : d->edge_u[e];
      const int64_t ph = p->node_pos[head];
      if (ph < 0 || (uint64_t)ph >= nf) continue;
      const int64_t pt = p->node_pos[tail];
      if (pt < 0) {
        delete p;
        return fail(THRML_EINVAL, "Node not found in global location map");
      }
      if (blk_of((uint64_t)pt) == blk_of((uint64_t)ph)) intra = true;
      slot_pos[fill[ph]] = (uint32_t)pt;
      slot_w[fill[ph]] = d->beta * d->weights[e];
      fill[ph]++;
    }
  }
  p->intra_block_edges = intra;
  plan_staging(p);
  std::vector<float> bias_w(nf);
  for (uint64_t k = 0; k < nf; ++k) bias_w[k] = d->beta * d->biases[p->pos_node[k]];

  std::vector<uint32_t> dir;
  if (!intra && one_per_block && detect_lattice(p, d->n_nodes, row_off, slot_pos, dir)) {
    p->kind = K_LATTICE;
    DevBuf d_dir, d_w, d_b;
    if ((rc = upload(p, p->row_off, row_off)) || (rc = upload(p, d_dir, dir)) ||
        (rc = upload(p, d_w, slot_w)) || (rc = upload(p, d_b, bias_w)) ||
        (rc = p->table.alloc(nf * 16 * sizeof(uint32_t)))) {
      delete p;
      return rc;
    }
    p->device_bytes += p->table.bytes;
    rc = launch_lattice_table(p, d_dir.as<uint32_t>(), d_w.as<float>(), d_b.as<float>());
    if (!rc) {
      hipError_t e = hipStreamSynchronize(ctx->stream);
      if (e != hipSuccess) rc = hip_fail(e, "lattice table");
    }
    p->device_bytes -= p->row_off.bytes + d_dir.bytes + d_w.bytes + d_b.bytes;
    p->row_off.release();
    if (rc) {
      delete p;
      return rc;
    }
  } else {
    p->kind = K_CSR;
    csr_windows(p, row_off);
    // 16 spare slots: the sweep kernel reads slot records in batches of 16
    std::vector<uint32_t> slots2(2 * (ns + 16), 0u);
    for (uint64_t s = 0; s < ns; ++s) {
      slots2[2 * s] = slot_pos[s];
      std::memcpy(&slots2[2 * s + 1], &slot_w[s], 4);
    }
    if ((rc = upload(p, p->row_off, row_off)) || (rc = upload(p, p->slots, slots2)) ||
        (rc = upload(p, p->bias_w, bias_w))) {
      delete p;
      return rc;
    }
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
      delete p;
      return hip_fail(e, "program upload");
    }
  }
  *out = p;
  return THRML_OK;
}

// FactorSamplingProgram over [bias factor, CategoricalEBMFactor([U, V], W)]
// with CategoricalGibbsConditional(q, 0) per free block
// (crates/thrml-models/src/factor.rs:152-185,
// crates/thrml-models/src/discrete_ebm.rs:456-548).  Slots of a free position:
// the edges where it is u (tail v, ascending e), then those where it is v
// (tail u, ascending e), the order in which program.rs:102-200 lays out the
// head-U and head-V groups.
extern "C" int thrml_potts_program_create(thrml_ctx *ctx, const thrml_potts_desc *d,
                                          thrml_prog **out) {
  if (!ctx || !d || !out) return fail(THRML_EINVAL, "NULL argument");
  if (d->q < 2 || d->q > POTTS_WIDE_MAX_Q) return fail(THRML_EINVAL, "q must lie in 2..65536");
  if (d->n_free_blocks == 0)
    return fail(THRML_EINVAL, "Number of samplers (0) must match number of free blocks (0)");
  if (d->n_edges && (!d->edge_u || !d->edge_v || !d->weights))
    return fail(THRML_EINVAL, "edge arrays are NULL");
  if (d->n_nodes && !d->biases) return fail(THRML_EINVAL, "biases is NULL");
  if (d->n_edges > 0x7fffffffull) return fail(THRML_EUNSUPPORTED, "more than 2^31-1 edges");
  if ((uint64_t)d->q * d->q * d->n_edges > (1ull << 40))
    return fail(THRML_EUNSUPPORTED, "the weights (edges x q x q floats) exceed 4 TiB");
  THRML_HIP(hipSetDevice(ctx->device));
  if (int rc = fast_math_gate(ctx, nullptr, nullptr)) return rc;
  auto *p = new thrml_prog();
  p->ctx = ctx;
  p->kind = K_POTTS;
  p->q = d->q;
  p->cat_bytes = p->q > POTTS_MAX_Q ? 2u : 1u;  // two bytes of state per node above 256
  p->n_edges = d->n_edges;
  int rc = build_blocks(p, d->n_nodes, d->n_free_blocks, d->free_offsets, d->free_nodes,
                        d->n_clamped_blocks, d->clamped_offsets, d->clamped_nodes);
  if (!rc) rc = set_superblocks(p, d->n_superblocks, d->superblock_offsets);
  if (rc) {
    delete p;
    return rc;
  }
  // slots for the free positions only; an edge between two clamped nodes
  // takes none (it enters the energies alone)
  const uint64_t nf = p->blk_off[p->n_free];
  const uint32_t q = d->q;
  std::vector<uint32_t> row_off(nf + 1, 0), nu(nf, 0);
  for (uint64_t e = 0; e < d->n_edges; ++e) {
    const uint32_t a = d->edge_u[e], b = d->edge_v[e];
    if (a >= d->n_nodes || b >= d->n_nodes || p->node_pos[a] < 0 || p->node_pos[b] < 0) {
      delete p;
      return fail(THRML_EINVAL, "Node not found in global location map");
    }
    const uint64_t pa = (uint64_t)p->node_pos[a], pb = (uint64_t)p->node_pos[b];
    if (pa < nf) {
      row_off[pa + 1]++;
      nu[pa]++;
    }
    if (pb < nf) row_off[pb + 1]++;
  }
  for (uint64_t k = 0; k < nf; ++k) row_off[k + 1] += row_off[k];
  std::vector<uint32_t> uend(nf), fu(nf), fv(nf);
  for (uint64_t k = 0; k < nf; ++k) {
    uend[k] = row_off[k] + nu[k];
    fu[k] = row_off[k];
    fv[k] = uend[k];
  }
  std::vector<uint32_t> slots(2 * (size_t)row_off[nf]);
  auto blk_of = [&](uint64_t pos) {
    return (uint32_t)(std::upper_bound(p->blk_off.begin(), p->blk_off.end(), pos) -
                      p->blk_off.begin() - 1);
  };
  bool intra = false;
  for (uint64_t e = 0; e < d->n_edges; ++e) {
    const uint32_t pu = (uint32_t)p->node_pos[d->edge_u[e]];
    const uint32_t pv = (uint32_t)p->node_pos[d->edge_v[e]];
    if (blk_of(pu) == blk_of(pv) && blk_of(pu) < p->n_free) intra = true;
    if (pu < nf) {
      slots[2 * (size_t)fu[pu]] = pv;
      slots[2 * (size_t)fu[pu] + 1] = (uint32_t)e;
      fu[pu]++;
    }
    if (pv < nf) {
      slots[2 * (size_t)fv[pv]] = pu;
      slots[2 * (size_t)fv[pv] + 1] = (uint32_t)e;
      fv[pv]++;
    }
  }
  p->intra_block_edges = intra;
  plan_staging(p);
  p->eu.assign(d->edge_u, d->edge_u + d->n_edges);  // for the energies
  p->ev.assign(d->edge_v, d->edge_v + d->n_edges);
  // per position (free and clamped: the energies read every position)
  std::vector<float> bias((size_t)p->n_total * q);
  for (uint64_t k = 0; k < p->n_total; ++k)
    for (uint32_t c = 0; c < q; ++c) bias[k * q + c] = 0.0f + d->biases[(size_t)p->pos_node[k] * q + c];
  // weights and their transpose (a u-role slot reads column x_v of W[e], row
  // x_v of W[e]^T); with q <= 16 an all-zero edge E is appended, the padding
  // slots' matrix in the role-padded kernel.  Wider kernels read only the
  // real slots' rows, so a q = 65536 program does not carry a 16 GiB pad.
  const size_t qq = (size_t)q * q;
  const size_t n_w = (d->n_edges + (q <= 16u ? 1u : 0u)) * qq;
  // (the caller's weights go to the device once; the transposed copy and the
  // padding edge are written there)
  // role-padded slot lists: M u-role slots then M v-role slots per position,
  // M = 2 or 4 (the smallest that holds every position's roles), padding
  // {own position, edge E}
  uint32_t mu = 0, mv = 0;
  for (uint64_t k = 0; k < nf; ++k) {
    mu = std::max(mu, uend[k] - row_off[k]);
    mv = std::max(mv, row_off[k + 1] - uend[k]);
  }
  const uint32_t m = std::max(mu, mv);
  p->mean_slots = nf ? (uint32_t)((row_off[nf] + nf / 2) / nf) : 0u;
  p->pm = (q % 4 == 0 && q <= 16 && d->n_edges > 0) ? (m <= 2 ? 2u : m <= 4 ? 4u : 0u) : 0u;
  std::vector<uint32_t> ps;
  if (p->pm) {
    const uint32_t M = p->pm;
    ps.assign(nf * 4 * M, 0u);
    for (uint64_t k = 0; k < nf; ++k) {
      uint32_t *r = &ps[k * 4 * M];
      for (uint32_t j = 0; j < 2 * M; ++j) {
        r[2 * j] = (uint32_t)k;
        r[2 * j + 1] = (uint32_t)d->n_edges;
      }
      for (uint32_t s = row_off[k], j = 0; s < uend[k]; ++s, ++j) {
        r[2 * j] = slots[2 * (size_t)s];
        r[2 * j + 1] = slots[2 * (size_t)s + 1];
      }
      for (uint32_t s = uend[k], j = M; s < row_off[k + 1]; ++s, ++j) {
        r[2 * j] = slots[2 * (size_t)s];
        r[2 * j + 1] = slots[2 * (size_t)s + 1];
      }
    }
  }
  if ((rc = upload(p, p->row_off, row_off)) || (rc = upload(p, p->uend, uend)) ||
      (rc = upload(p, p->slots, slots)) || (rc = upload(p, p->bias_w, bias)) ||
      (rc = p->wts.alloc(n_w * sizeof(float))) || (rc = p->wts_t.alloc(n_w * sizeof(float))) ||
      (p->pm && (rc = upload(p, p->pslots, ps)))) {
    (void)hipStreamSynchronize(ctx->stream);
    delete p;
    return rc;
  }
  p->device_bytes += p->wts.bytes + p->wts_t.bytes;
  if (d->n_edges) {
    const hipError_t ew = hipMemcpyAsync(p->wts.p, d->weights, d->n_edges * qq * sizeof(float),
                                         hipMemcpyHostToDevice, ctx->stream);
    if (ew != hipSuccess) {
      (void)hipStreamSynchronize(ctx->stream);
      delete p;
      return hip_fail(ew, "program upload");
    }
  }
  if ((rc = launch_potts_weights(ctx, p->wts.as<float>(), p->wts_t.as<float>(), d->n_edges, q, n_w))) {
    (void)hipStreamSynchronize(ctx->stream);
    delete p;
    return rc;
  }
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    delete p;
    return hip_fail(e, "program upload");
  }
  *out = p;
  return THRML_OK;
}

// FactorSamplingProgram over DiscreteEBMFactors (crates/thrml-models/src/factor.rs:
// 126-185).  Interaction groups per factor in order (to_interaction_groups,
// crates/thrml-models/src/discrete_ebm.rs:371-540): with spin groups, one group
// whose head is spin group 0 ++ ... ++ spin group n_spin-1 (head position
// j = i * batch + b; tails: the other spin groups ascending, then every
// categorical group; weight row b); then one group per categorical group h
// (head position b; tails: every spin group, then the other categorical group;
// the weight row with axis h first).  Slots of a free position: groups in
// order, head positions ascending (crates/thrml-samplers/src/program.rs:102-200).
namespace {

// A factor's weights in the device array: rows as given at w_base, and for a
// factor with two categorical groups a transposed copy ([b][d2][d1]) at
// wt_base, which the head-U slots read so that every categorical head reads
// one contiguous row of q weights.  Bases are multiples of 4 floats.
struct DiscFactor {
  const thrml_discrete_factor *f;
  uint64_t w_base, wt_base;
};

// Checks of (Square)DiscreteEBMFactor::new (discrete_ebm.rs:300-358, 862-885) and of what the
// two conditionals read of a factor's weights.
int check_factor(const thrml_discrete_desc *d, const thrml_discrete_factor &F, uint32_t q) {
  // SquareDiscreteEBMFactor::new checks the shape first (discrete_ebm.rs:868-877)
  if (F.flags & ~THRML_FACTOR_SQUARE) return fail(THRML_EINVAL, "unknown factor flags");
  if ((F.flags & THRML_FACTOR_SQUARE) && F.d1 != F.d2)
    return fail(THRML_EINVAL, "Interaction tensor is not square");
  const uint32_t ng = F.n_spin_groups + F.n_cat_groups;
  if (ng == 0) return fail(THRML_EINVAL, "At least one node group must be provided");
  if (F.n_cat_groups > 2)
    return fail(THRML_EINVAL, "weights are [b, d1, d2]: at most two categorical node groups");
  if (F.n_spin_groups > 255) return fail(THRML_EUNSUPPORTED, "at most 255 spin node groups per factor");
  if (F.batch == 0) return fail(THRML_EINVAL, "Block cannot be empty");
  if (F.d1 == 0 || F.d2 == 0) return fail(THRML_EINVAL, "weight dimensions must be positive");
  if (!F.nodes || !F.weights) return fail(THRML_EINVAL, "factor arrays are NULL");
  const uint32_t eff = F.d2 > 1 ? 2u : (F.d1 > 1 ? 1u : 0u);  // trailing 1s dropped
  if (eff < F.n_cat_groups)
    return fail(THRML_EINVAL,
                "The shape of the weight tensor must be [b, x_1, ..., x_k], where k is the length "
                "of categorical_node_groups (" + std::to_string(F.n_cat_groups) +
                    "). Got effective dims: " + std::to_string(eff));
  for (uint32_t g = 0; g < ng; ++g)
    for (uint32_t b = 0; b < F.batch; ++b) {
      const uint32_t node = F.nodes[(size_t)g * F.batch + b];
      if (node >= d->n_nodes) return fail(THRML_EINVAL, "Node not found in global location map");
      if ((d->node_kind[node] != 0) != (g >= F.n_spin_groups))
        return fail(THRML_EINVAL,
                    "spin node groups must hold spin nodes and categorical node groups "
                    "categorical nodes");
    }
  const uint64_t dd = (uint64_t)F.d1 * F.d2;
  if (F.n_spin_groups && F.n_cat_groups == 0 && dd != 1)
    return fail(THRML_EINVAL, "a spin factor without categorical groups has weights [b, 1, 1]");
  if (F.n_spin_groups && F.n_cat_groups && dd < q)
    return fail(THRML_EINVAL, "a spin head indexes its weight row by a category: d1 * d2 >= q");
  if (F.n_cat_groups == 1 && dd != q)
    return fail(THRML_EINVAL, "a factor with one categorical group has weights [b, q, 1]");
  if (F.n_cat_groups == 2 && (F.d1 != q || F.d2 != q))
    return fail(THRML_EINVAL, "a factor with two categorical groups has weights [b, q, q]");
  return THRML_OK;
}

}  // namespace

extern "C" int thrml_discrete_program_create(thrml_ctx *ctx, const thrml_discrete_desc *d,
                                             thrml_prog **out) {
  if (!ctx || !d || !out) return fail(THRML_EINVAL, "NULL argument");
  if (d->n_free_blocks == 0)
    return fail(THRML_EINVAL, "Number of samplers (0) must match number of free blocks (0)");
  if (d->n_nodes && !d->node_kind) return fail(THRML_EINVAL, "node_kind is NULL");
  if (d->n_factors && !d->factors) return fail(THRML_EINVAL, "factors is NULL");
  bool any_cat = false;
  for (uint32_t x = 0; x < d->n_nodes; ++x) any_cat |= d->node_kind[x] != 0;
  if (any_cat && (d->q < 2 || d->q > POTTS_WIDE_MAX_Q))
    return fail(THRML_EINVAL, "q must lie in 2..65536");
  THRML_HIP(hipSetDevice(ctx->device));
  if (int rc = fast_math_gate(ctx, nullptr, nullptr)) return rc;
  auto *p = new thrml_prog();
  p->ctx = ctx;
  p->kind = K_DISCRETE;
  p->q = any_cat ? d->q : 2u;
  p->cat_bytes = p->q > POTTS_MAX_Q ? 2u : 1u;  // two bytes of state per node above 256
  auto bail = [&](int rc) {
    delete p;
    return rc;
  };
  int rc = build_blocks(p, d->n_nodes, d->n_free_blocks, d->free_offsets, d->free_nodes,
                        d->n_clamped_blocks, d->clamped_offsets, d->clamped_nodes);
  if (!rc) rc = set_superblocks(p, d->n_superblocks, d->superblock_offsets);
  if (rc) return bail(rc);
  const uint32_t nb = p->n_free + p->n_clamped;
  p->blk_kind.assign(nb, 0);
  for (uint32_t b = 0; b < nb; ++b)
    for (uint64_t k = p->blk_off[b]; k < p->blk_off[b + 1]; ++k) {
      const uint8_t kind = d->node_kind[p->pos_node[k]] ? 1 : 0;
      if (k == p->blk_off[b])
        p->blk_kind[b] = kind;
      else if (kind != p->blk_kind[b])
        return bail(fail(THRML_EINVAL, "a block holds both spin and categorical nodes"));
    }
  const uint32_t q = p->q;
  std::vector<DiscFactor> fs(d->n_factors);
  uint64_t n_w = 0;
  for (uint32_t i = 0; i < d->n_factors; ++i) {
    const thrml_discrete_factor &F = d->factors[i];
    if ((rc = check_factor(d, F, q))) return bail(rc);
    const uint64_t sz = (uint64_t)F.batch * F.d1 * F.d2;
    fs[i].f = &F;
    fs[i].w_base = n_w;
    n_w = (n_w + sz + 3u) & ~3ull;
    fs[i].wt_base = n_w;
    if (F.n_cat_groups == 2) n_w = (n_w + sz + 3u) & ~3ull;
  }
  if (n_w >= 0xffffffffull) return bail(fail(THRML_EUNSUPPORTED, "more than 2^32-1 factor weights"));
  // at least 16 floats: a slot past a site's last one (the sweep reads the
  // spare record below) reads entries 0..15 of the array and adds nothing
  std::vector<float> w(std::max<uint64_t>(n_w, 16), 0.0f);
  for (const DiscFactor &df : fs) {
    const thrml_discrete_factor &F = *df.f;
    std::copy(F.weights, F.weights + (size_t)F.batch * F.d1 * F.d2, w.begin() + (long)df.w_base);
    if (F.n_cat_groups == 2)
      for (uint64_t b = 0; b < F.batch; ++b)
        for (uint32_t c = 0; c < F.d1; ++c)
          for (uint32_t x = 0; x < F.d2; ++x)
            w[df.wt_base + (b * F.d2 + x) * F.d1 + c] = F.weights[(b * F.d1 + c) * F.d2 + x];
  }

  // slots: a counting pass, then a filling pass
  const uint64_t nf = p->blk_off[p->n_free];
  std::vector<uint32_t> row_off(nf + 1, 0), cursor, slots, sp, last(nf, DISC_NONE);
  auto blk_of = [&](uint64_t pos) {
    return (uint32_t)(std::upper_bound(p->blk_off.begin(), p->blk_off.end(), pos) - p->blk_off.begin() - 1);
  };
  bool intra = false;
  for (int pass = 0; pass < 2; ++pass) {
    if (pass == 1) {
      for (uint64_t k = 0; k < nf; ++k) row_off[k + 1] += row_off[k];
      if (row_off[nf] == DISC_NONE) return bail(fail(THRML_EUNSUPPORTED, "too many slots"));
      cursor.assign(row_off.begin(), row_off.end() - 1);
      // one spare record at the end: weight offset 0, no tails
      slots.assign(4 * (size_t)row_off[nf] + 4, 0u);
      slots[4 * (size_t)row_off[nf] + 1] = DISC_NONE;
    }
    uint32_t group = 0;
    for (const DiscFactor &df : fs) {
      const thrml_discrete_factor &F = *df.f;
      const uint32_t B = F.batch, ns = F.n_spin_groups, nc = F.n_cat_groups;
      const uint32_t n_heads = (ns ? 1u : 0u) + nc;
      for (uint32_t hg = 0; hg < n_heads; ++hg, ++group) {
        const bool spin_head = ns && hg == 0;
        const uint32_t h = ns ? hg - 1 : hg;
        // a square factor's two categorical-head groups are one merged group
        const uint32_t gid = (F.flags & THRML_FACTOR_SQUARE) && !spin_head && h == 1 ? group - 1 : group;
        const uint64_t n_j = spin_head ? (uint64_t)ns * B : B;
        for (uint64_t j = 0; j < n_j; ++j) {
          const uint32_t hi = spin_head ? (uint32_t)(j / B) : h;
          const uint32_t b = spin_head ? (uint32_t)(j % B) : (uint32_t)j;
          const uint32_t head = F.nodes[(size_t)(spin_head ? hi : ns + h) * B + b];
          const int64_t hp = p->node_pos[head];
          if (hp < 0 || (uint64_t)hp >= nf) continue;
          // tails: spin groups (minus the head's own for a spin head), then
          // categorical groups (minus the head's for a categorical head);
          // the first categorical tail is the one the conditionals read
          uint32_t n_sp = 0, cat = DISC_NONE;
          const uint32_t sp_beg = (uint32_t)sp.size();
          for (uint32_t k = 0; k < ns + nc; ++k) {
            if (spin_head ? k == hi : k == ns + h) continue;
            const int64_t tp = p->node_pos[F.nodes[(size_t)k * B + b]];
            if (tp < 0) return bail(fail(THRML_EINVAL, "Node not found in global location map"));
            const bool read = k < ns || cat == DISC_NONE;
            if (read && blk_of((uint64_t)tp) == blk_of((uint64_t)hp)) intra = true;
            if (k < ns) {
              ++n_sp;
              if (pass == 1) sp.push_back((uint32_t)tp);
            } else if (cat == DISC_NONE) {
              cat = (uint32_t)tp;
            }
          }
          if (pass == 0) {
            row_off[hp + 1]++;
            continue;
          }
          // head U (h = 0) reads W[b][c][x_V], row x_V of the transposed copy
          const uint32_t axis = spin_head || cat == DISC_NONE ? 0u : 2u;
          const bool tr = !spin_head && cat != DISC_NONE && h == 0;
          const uint32_t first = last[hp] != gid ? 1u : 0u;
          last[hp] = gid;
          uint32_t *r = &slots[4 * (size_t)cursor[hp]++];
          r[0] = (uint32_t)((tr ? df.wt_base : df.w_base) + (uint64_t)b * F.d1 * F.d2);
          r[1] = cat;
          r[2] = sp_beg;
          r[3] = n_sp | first << 8 | axis << 9;
        }
      }
    }
  }
  if (sp.size() >= DISC_NONE) return bail(fail(THRML_EUNSUPPORTED, "too many spin tails"));
  p->intra_block_edges = intra;
  plan_staging(p);

  // energy terms: factor rows whose nodes all have a position
  std::vector<uint32_t> terms, tsp;
  for (const DiscFactor &df : fs) {
    const thrml_discrete_factor &F = *df.f;
    const uint32_t B = F.batch, ns = F.n_spin_groups, nc = F.n_cat_groups;
    for (uint32_t b = 0; b < B; ++b) {
      bool all = true;
      for (uint32_t k = 0; k < ns + nc && all; ++k) all = p->node_pos[F.nodes[(size_t)k * B + b]] >= 0;
      if (!all) continue;
      const uint32_t t0 = (uint32_t)tsp.size();
      for (uint32_t k = 0; k < ns; ++k) tsp.push_back((uint32_t)p->node_pos[F.nodes[(size_t)k * B + b]]);
      const uint32_t x0 = nc > 0 ? (uint32_t)p->node_pos[F.nodes[(size_t)ns * B + b]] : DISC_NONE;
      const uint32_t x1 = nc > 1 ? (uint32_t)p->node_pos[F.nodes[(size_t)(ns + 1) * B + b]] : DISC_NONE;
      const uint32_t rec[8] = {(uint32_t)(df.w_base + (uint64_t)b * F.d1 * F.d2), t0, ns, x0,
                               x1, F.d2, 0u, 0u};
      terms.insert(terms.end(), rec, rec + 8);
    }
  }
  if (tsp.size() >= DISC_NONE) return bail(fail(THRML_EUNSUPPORTED, "too many energy terms"));
  p->d_nterms = terms.size() / 8;
  if (sp.empty()) sp.push_back(0u);
  if (tsp.empty()) tsp.push_back(0u);
  if (terms.empty()) terms.assign(8, 0u);
  if ((rc = upload(p, p->row_off, row_off)) || (rc = upload(p, p->d_slots, slots)) ||
      (rc = upload(p, p->d_sp, sp)) || (rc = upload(p, p->d_w, w)) ||
      (rc = upload(p, p->d_terms, terms)) || (rc = upload(p, p->d_tsp, tsp)))
    return bail(rc);
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return bail(hip_fail(e, "program upload"));
  *out = p;
  return THRML_OK;
}

extern "C" void thrml_prog_destroy(thrml_prog *p) {
  if (!p) return;
  (void)hipSetDevice(p->ctx->device);
  (void)hipStreamSynchronize(p->ctx->stream);
  delete p;
}

extern "C" int thrml_prog_get_info(const thrml_prog *p, thrml_prog_info *o) {
  if (!p || !o) return fail(THRML_EINVAL, "NULL argument");
  o->kind = p->kind;
  o->n_free_blocks = p->n_free;
  o->n_clamped_blocks = p->n_clamped;
  o->n_total = p->n_total;
  o->device_bytes = p->device_bytes;
  o->dense_pieces = p->kind == K_DENSE ? p->dense_pieces : 0u;
  return THRML_OK;
}

extern "C" int thrml_prog_block(const thrml_prog *p, uint32_t b, uint64_t *offset, uint64_t *len) {
  if (!p) return fail(THRML_EINVAL, "NULL program");
  if (b >= p->n_free + p->n_clamped) return fail(THRML_EINVAL, "block index out of range");
  if (offset) *offset = p->blk_off[b];
  if (len) *len = p->blk_off[b + 1] - p->blk_off[b];
  return THRML_OK;
}

// ---------------------------------------------------------------------------
// states
extern "C" int thrml_state_create(thrml_prog *p, uint32_t n_chains, thrml_state **out) {
  if (!p || !out) return fail(THRML_EINVAL, "NULL argument");
  if (n_chains == 0) return fail(THRML_EINVAL, "n_chains must be positive");
  THRML_HIP(hipSetDevice(p->ctx->device));
  auto *st = new thrml_state();
  st->prog = p;
  st->ctx = p->ctx;
  st->C = n_chains;
  st->G = (n_chains + 63u) / 64u;
  st->Cp = (n_chains + 3u) / 4u * 4u;
  const bool cat = byte_layout(p);
  DevBuf &buf = cat ? st->cat : st->words;
  const size_t bytes = cat ? (size_t)st->Cp * p->n_total * p->cat_bytes
                           : (size_t)st->G * p->planes * p->n_total * sizeof(uint64_t);
  int rc = buf.alloc(bytes);
  if (!rc) {
    hipError_t e = hipMemsetAsync(buf.p, 0, bytes, p->ctx->stream);
    if (e != hipSuccess) rc = hip_fail(e, "hipMemsetAsync");
  }
  if (!rc) rc = st->flag.alloc(sizeof(uint32_t));
  // the sweep kernel's half-size gather copy (refreshed at each run's start)
  if (!rc && p->kind == K_CSR && n_chains <= 32u && p->planes == 1u && p->stage_max == 0)
    rc = st->low.alloc((size_t)p->n_total * sizeof(uint32_t));
  if (!rc && p->stage_max) {
    // cleared once: the padding chains of a categorical row are copied back
    // with the staged range but never written
    rc = st->scratch.alloc(cat ? (size_t)st->Cp * p->stage_max * p->cat_bytes
                               : (size_t)st->G * p->planes * p->stage_max * sizeof(uint64_t));
    if (!rc) {
      hipError_t e = hipMemsetAsync(st->scratch.p, 0, st->scratch.bytes, p->ctx->stream);
      if (e != hipSuccess) rc = hip_fail(e, "hipMemsetAsync");
    }
  }
  if (!rc && p->kind == K_DENSE) {
    st->C_pad = (n_chains + 255u) / 256u * 256u;
    rc = st->dbits_v.alloc((size_t)st->C_pad * (p->Vp / 32) * 4);
    if (!rc) rc = st->dbits_h.alloc((size_t)st->C_pad * (p->Hp / 32) * 4);
    if (!rc) rc = launch_dense_sync_act(st, 0);
    if (!rc) rc = launch_dense_sync_act(st, 1);
  }
  if (!rc) {
    hipError_t e = hipStreamSynchronize(p->ctx->stream);
    if (e != hipSuccess) rc = hip_fail(e, "state allocation");
  }
  if (rc) {
    delete st;
    return rc;
  }
  *out = st;
  return THRML_OK;
}

extern "C" void thrml_state_destroy(thrml_state *st) {
  if (!st) return;
  (void)hipSetDevice(st->ctx->device);
  (void)hipStreamSynchronize(st->ctx->stream);
  delete st;
}

// The context whose observer callback this thread is running (a run started
// from inside it would reuse the context's key store and lock, and a state
// write would change the chains between two sweeps of the run).
static thread_local const thrml_ctx *tl_observing = nullptr;
static int not_observing(const thrml_ctx *ctx) {
  if (tl_observing == ctx)
    return fail(THRML_EINVAL, "a run cannot start inside an observer callback on the same context");
  return THRML_OK;
}
// Marks ctx as observing for one callback; the previous mark comes back on
// any exit, so an observer that runs another context's observer keeps its
// own guard, and an exception thrown through the callback leaves no mark.
struct ObservingScope {
  const thrml_ctx *prev;
  explicit ObservingScope(const thrml_ctx *ctx) : prev(tl_observing) { tl_observing = ctx; }
  ~ObservingScope() { tl_observing = prev; }
  ObservingScope(const ObservingScope &) = delete;
  ObservingScope &operator=(const ObservingScope &) = delete;
};

static int state_io(thrml_state *st, uint32_t b, void *buf, int dtype, int on_device, bool write) {
  if (!st || !buf) return fail(THRML_EINVAL, "NULL argument");
  thrml_prog *p = st->prog;
  if (b >= p->n_free + p->n_clamped) return fail(THRML_EINVAL, "block index out of range");
  if (dtype != THRML_DTYPE_U8 && dtype != THRML_DTYPE_F32) return fail(THRML_EINVAL, "unknown dtype");
  if (!write && dtype == THRML_DTYPE_U8 && p->cat_bytes == 2)
    return fail(THRML_EINVAL, "categories above 255 do not fit the u8 dtype: read this state as f32");
  if (write && tl_observing == p->ctx)
    return fail(THRML_EINVAL, "a state cannot be written inside an observer callback on its context");
  THRML_HIP(hipSetDevice(p->ctx->device));
  const size_t n = (size_t)st->C * (p->blk_off[b + 1] - p->blk_off[b]);
  const size_t bytes = n * (dtype == THRML_DTYPE_U8 ? 1 : 4);
  void *dev = buf;
  DevBuf tmp;
  if (!on_device) {
    if (int rc = tmp.alloc(bytes)) return rc;
    dev = tmp.p;
    if (write) THRML_HIP(hipMemcpyAsync(dev, buf, bytes, hipMemcpyHostToDevice, p->ctx->stream));
  }
  int rc;
  uint32_t *bad = st->flag.as<uint32_t>();
  if (write) {
    // every value is checked before the block is written, so a rejected
    // import leaves the state as it was
    const uint32_t q = byte_layout(p) ? block_q(p, b) : 2u;
    uint32_t bad_h = 0;
    THRML_HIP(hipMemsetAsync(bad, 0, sizeof(uint32_t), p->ctx->stream));
    if ((rc = launch_import_check(p->ctx, dev, dtype, n, q, bad))) return rc;
    THRML_HIP(hipMemcpyAsync(&bad_h, bad, sizeof(uint32_t), hipMemcpyDeviceToHost, p->ctx->stream));
    THRML_HIP(hipStreamSynchronize(p->ctx->stream));
    if (bad_h) {
      if (q > 2 || p->kind == K_POTTS)
        return fail(THRML_EINVAL, "category value out of range: block " + std::to_string(b) +
                                      " holds a value outside 0.." + std::to_string(q - 1) +
                                      " (the state is unchanged)");
      return fail(THRML_EINVAL, "spin value out of range: block " + std::to_string(b) +
                                    " holds a value other than 0 and 1 (the state is unchanged)");
    }
  }
  if (byte_layout(p))
    rc = write ? launch_potts_pack(st, b, dev, dtype, bad) : launch_potts_unpack(st, b, dev, dtype);
  else
    rc = write ? launch_pack(st, b, dev, dtype, bad) : launch_unpack(st, b, dev, dtype);
  if (!rc && write && p->kind == K_DENSE) rc = launch_dense_sync_act(st, p->dense_side[b]);
  if (rc) return rc;
  if (!write && !on_device)
    THRML_HIP(hipMemcpyAsync(buf, dev, bytes, hipMemcpyDeviceToHost, p->ctx->stream));
  if (write || !on_device) THRML_HIP(hipStreamSynchronize(p->ctx->stream));  // tmp is freed on return
  return THRML_OK;
}

extern "C" int thrml_state_set_block(thrml_state *st, uint32_t b, const void *src, int dtype,
                                     int src_on_device) {
  return state_io(st, b, const_cast<void *>(src), dtype, src_on_device, true);
}

extern "C" int thrml_state_get_block(thrml_state *st, uint32_t b, void *dst, int dtype,
                                     int dst_on_device) {
  return state_io(st, b, dst, dtype, dst_on_device, false);
}

// ---------------------------------------------------------------------------
// sweep drivers
namespace {

int half_sweep(thrml_prog *p, thrml_state *st, uint32_t b, const uint32_t *keys,
               const LatticeMoments *mom) {
  switch (p->kind) {
    case K_LATTICE: return launch_lattice_half(p, st, b, keys, mom);
    case K_CSR: return launch_csr_half(p, st, b, keys);
    case K_POTTS: return launch_potts_half(p, st, b, keys);
    case K_DENSE: return launch_dense_half(p, st, p->dense_side[b], keys);
    case K_DISCRETE: return launch_discrete_half(p, st, b, keys);
  }
  return fail(THRML_EINVAL, "unknown program kind");
}

// A run: the key tree, the number of sweeps and the observation points
// (observation k follows sweep obs_after[k]; -1 = before the first sweep).
struct Plan {
  KeyPlan kp;
  uint64_t n_sweeps = 0;
  std::vector<int64_t> obs_after;
};

Plan blocks_plan(thrml_prog *p, thrml_state *st, uint64_t key, uint64_t n_iters) {
  Plan pl;
  pl.kp = KeyPlan{key, st->C, st->G * 64u, p->n_free, 0u, n_iters, 0, 0, 0};
  pl.n_sweeps = n_iters;
  return pl;
}

// sample_with_observation's schedule (crates/thrml-samplers/src/sampling.rs:178-320):
// n_warmup sweeps, observation, then n_samples-1 times (steps_per_sample
// sweeps, observation).
Plan schedule_plan(thrml_prog *p, thrml_state *st, uint64_t key, const thrml_schedule &s) {
  Plan pl;
  pl.kp = KeyPlan{key, st->C, st->G * 64u, p->n_free, 1u, 0, s.n_warmup, s.n_samples,
                  s.steps_per_sample};
  pl.n_sweeps = s.n_warmup + (s.n_samples > 1 ? (s.n_samples - 1) * s.steps_per_sample : 0);
  pl.obs_after.push_back((int64_t)s.n_warmup - 1);
  for (uint64_t i = 0; i + 1 < s.n_samples; ++i)
    pl.obs_after.push_back((int64_t)(s.n_warmup + (i + 1) * s.steps_per_sample) - 1);
  return pl;
}

// Where a run keeps its expanded stream keys: a growable device buffer (the
// context's), or a fixed region of cap bytes.
struct KeyStore {
  DevBuf *grow = nullptr;
  uint32_t *fixed = nullptr;
  uint64_t cap = 0;
};

// Bytes of expanded stream keys one sweep of st needs.
uint64_t key_bytes_per_sweep(const thrml_prog *p, const thrml_state *st) {
  return (uint64_t)p->n_free * st->G * 64u * KEY_WORDS * sizeof(uint32_t);
}

// Runs the plan.  obs(fused) is called at each observation; fused = true when
// the sweep before it already added the observation to `fuse`'s counters.
// The keys are computed in chunks of sweeps that fit the key store.
template <class Obs>
int run_plan(thrml_prog *p, thrml_state *st, const Plan &pl, const LatticeMoments *fuse, Obs obs,
             const KeyStore &ks) {
  const uint32_t B = p->n_free;
  const uint64_t per_sweep = key_bytes_per_sweep(p, st);
  const uint64_t budget = ks.grow ? 64ull << 20 : ks.cap;
  if (per_sweep > budget) return fail(THRML_EINVAL, "one sweep's stream keys exceed the key store");
  const uint64_t chunk = std::max<uint64_t>(1, std::min<uint64_t>(budget / per_sweep, 1u << 20));
  const bool can_fuse = fuse && p->kind == K_LATTICE;
  size_t oi = 0;
  const size_t n_obs = pl.obs_after.size();
  while (oi < n_obs && pl.obs_after[oi] < 0) {
    if (int rc = obs(false)) return rc;
    ++oi;
  }
  // the words may have changed since the last run (state writes, hinton_init);
  // the sweeps keep the copy in step from here on
  if (pl.n_sweeps && st->low.p)
    if (int rc = launch_pack_low(st)) return rc;
  for (uint64_t s0 = 0; s0 < pl.n_sweeps; s0 += chunk) {
    const uint32_t ns = (uint32_t)std::min<uint64_t>(chunk, pl.n_sweeps - s0);
    const uint64_t need = ns * per_sweep;
    if (ks.grow && ks.grow->bytes < need) {
      THRML_HIP(hipStreamSynchronize(p->ctx->stream));
      if (int rc = ks.grow->alloc(need)) return rc;
    }
    uint32_t *keys = ks.grow ? ks.grow->as<uint32_t>() : ks.fixed;
    // the previous chunk's sweeps read the same buffer; stream order keeps
    // this launch behind them
    if (int rc = launch_key_schedule(p->ctx, pl.kp, s0, ns, keys)) return rc;
    for (uint32_t k = 0; k < ns; ++k) {
      const int64_t s = (int64_t)(s0 + k);
      const bool observed = oi < n_obs && pl.obs_after[oi] == s;
      const LatticeMoments *m = (observed && can_fuse) ? fuse : nullptr;
      // sample_blocks (crates/thrml-samplers/src/sampling.rs:28-63): the
      // superblocks in order, each block of one from the state before it
      for (uint32_t sb = 0; sb + 1 < p->sb_off.size(); ++sb) {
        for (uint32_t b = p->sb_off[sb]; b < p->sb_off[sb + 1]; ++b) {
          const uint32_t *kb = keys + ((size_t)k * B + b) * (size_t)st->G * 64u * KEY_WORDS;
          if (int rc = half_sweep(p, st, b, kb, m)) return rc;
        }
        if (int rc = commit_superblock(p, st, sb)) return rc;
      }
      bool fused = m != nullptr;
      while (oi < n_obs && pl.obs_after[oi] == s) {
        if (int rc = obs(fused)) return rc;
        fused = false;
        ++oi;
      }
    }
  }
  return THRML_OK;
}

// Position of every requested pair in the lattice edge counters
// (LatticeMoments::diff), or false if some pair is not a lattice edge.
bool lattice_pair_slots(const thrml_prog *p, const std::vector<uint32_t> &ppos,
                        std::vector<uint32_t> &slot) {
  const uint64_t n_b = (uint64_t)p->L * p->half;
  slot.resize(ppos.size() / 2);
  for (size_t k = 0; k < slot.size(); ++k) {
    uint64_t a = ppos[2 * k], b = ppos[2 * k + 1];
    if ((a >= n_b) == (b >= n_b)) return false;
    if (a < n_b) std::swap(a, b);  // a in block 1
    const uint64_t i = a - n_b, r = i / p->half, t = i % p->half;
    const uint64_t pp = (r + p->parity[1]) & 1u;
    const uint64_t nb[4] = {r * p->half + (t + pp == 0 ? p->half - 1 : t + pp - 1),
                            r * p->half + (t + pp == p->half ? 0 : t + pp),
                            (r == 0 ? p->L - 1 : r - 1) * p->half + t,
                            (r + 1 == p->L ? 0 : r + 1) * p->half + t};
    int d = -1;
    for (int q = 0; q < 4; ++q)
      if (nb[q] == b) d = q;
    if (d < 0) return false;
    slot[k] = (uint32_t)(i * 4 + (uint64_t)d);
  }
  return true;
}

}  // namespace

extern "C" int thrml_run_blocks(thrml_prog *p, uint64_t key, thrml_state *st, uint64_t n_iters) {
  if (!p || !st) return fail(THRML_EINVAL, "NULL argument");
  if (st->prog != p) return fail(THRML_EINVAL, "state belongs to another program");
  if (n_iters == 0) return THRML_OK;  // sampling.rs:89-91
  THRML_HIP(hipSetDevice(p->ctx->device));
  if (int rc = not_observing(p->ctx)) return rc;
  std::lock_guard<std::mutex> lk(p->ctx->run_mu);
  KeyStore ks;
  ks.grow = &p->ctx->keys;
  return run_plan(p, st, blocks_plan(p, st, key, n_iters), nullptr,
                  [](bool) { return THRML_OK; }, ks);
}

extern "C" int thrml_run_blocks_noalloc(thrml_prog *p, uint64_t key, thrml_state *st,
                                        uint64_t n_iters) {
  if (!p || !st) return fail(THRML_EINVAL, "NULL argument");
  if (st->prog != p) return fail(THRML_EINVAL, "state belongs to another program");
  const uint64_t need = key_bytes_per_sweep(p, st);
  if (need > THRML_NOALLOC_KEY_BYTES)
    return fail(THRML_EINVAL,
                "thrml_run_blocks_noalloc: one sweep needs " + std::to_string(need) +
                    " bytes of stream keys (free blocks x 64 ceil(chains / 64) x " +
                    std::to_string(KEY_WORDS * sizeof(uint32_t)) + "), above the fixed " +
                    std::to_string((uint64_t)THRML_NOALLOC_KEY_BYTES) +
                    " (THRML_NOALLOC_KEY_BYTES); use thrml_run_blocks");
  if (p->ctx->timing)
    return fail(THRML_EINVAL,
                "thrml_run_blocks_noalloc: kernel timing is on for this context (it creates "
                "HIP events per launch); turn it off with thrml_ctx_enable_timing(ctx, 0)");
  if (n_iters == 0) return THRML_OK;  // sampling.rs:89-91
  const int dev = p->ctx->device;
  if (dev >= kMaxDevices)
    return fail(THRML_EUNSUPPORTED, "thrml_run_blocks_noalloc: device ordinal " +
                                        std::to_string(dev) + " is above the 64 it supports");
  const ScratchSlot slot = scratch_slot(dev);
  if (!slot.done || !slot.ptr)
    return fail(THRML_EHIP, std::string("thrml_run_blocks_noalloc: the key array of device ") +
                                std::to_string(dev) + " was not set up (" +
                                hipGetErrorString(slot.err) +
                                "); it is tried again at the next thrml_ctx_create");
  THRML_HIP(hipSetDevice(dev));
  // one call at a time per GPU (the array is shared by every context on it),
  // and in GPU order: a call on another stream than the last waits for the
  // last call's work first
  std::lock_guard<std::mutex> use(g_scratch_use_mu[dev]);
  if (int rc = not_observing(p->ctx)) return rc;
  std::lock_guard<std::mutex> lk(p->ctx->run_mu);
  hipStream_t stream = p->ctx->stream;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  THRML_HIP(hipStreamIsCapturing(stream, &cs));
  const bool capturing = cs != hipStreamCaptureStatusNone;
  ScratchSlot &gs = g_scratch[dev];  // `last` is read and written under use_mu only
  if (!capturing && gs.last && gs.last != stream)
    THRML_HIP(hipStreamWaitEvent(stream, slot.done_ev, 0));
  KeyStore ks;
  ks.fixed = slot.ptr;
  ks.cap = THRML_NOALLOC_KEY_BYTES;
  const int rc = run_plan(p, st, blocks_plan(p, st, key, n_iters), nullptr,
                          [](bool) { return THRML_OK; }, ks);
  if (!capturing) {
    THRML_HIP(hipEventRecord(slot.done_ev, stream));
    gs.last = stream;
  }
  return rc;
}

extern "C" int thrml_moments_create(thrml_prog *p, const uint32_t *nodes, uint64_t n1,
                                    const uint32_t *pairs, uint64_t n2, thrml_moments **out) {
  if (!p || !out || (n1 && !nodes) || (n2 && !pairs)) return fail(THRML_EINVAL, "NULL argument");
  if (byte_layout(p)) return fail(THRML_EINVAL, "moments are defined for Ising programs");
  THRML_HIP(hipSetDevice(p->ctx->device));
  std::vector<uint32_t> npos(n1), ppos(2 * n2);
  for (uint64_t k = 0; k < n1; ++k) {
    if (nodes[k] >= p->node_pos.size() || p->node_pos[nodes[k]] < 0)
      return fail(THRML_EINVAL, "Node not found in global location map");
    npos[k] = (uint32_t)p->node_pos[nodes[k]];
  }
  for (uint64_t k = 0; k < 2 * n2; ++k) {
    if (pairs[k] >= p->node_pos.size() || p->node_pos[pairs[k]] < 0)
      return fail(THRML_EINVAL, "Node not found in global location map");
    ppos[k] = (uint32_t)p->node_pos[pairs[k]];
  }
  auto *m = new thrml_moments();
  m->prog = p;
  m->ctx = p->ctx;
  m->n1 = n1;
  m->n2 = n2;
  // Lattice programs count in the sweep kernels' own layout when every pair
  // is a lattice edge; otherwise counts are gathered per requested entry.
  std::vector<uint32_t> pslot;
  m->native = p->kind == K_LATTICE && lattice_pair_slots(p, ppos, pslot);
  m->len1 = m->native ? p->n_total : n1;
  m->len2 = m->native ? (uint64_t)p->L * p->half * 4u : n2;
  int rc;
  if (m->native) {
    if ((rc = upload_to(p->ctx, m->slot1, npos)) || (rc = upload_to(p->ctx, m->slot2, pslot))) {
      delete m;
      return rc;
    }
  } else if ((rc = upload_to(p->ctx, m->npos, npos)) || (rc = upload_to(p->ctx, m->ppos, ppos))) {
    delete m;
    return rc;
  }
  if ((rc = m->cnt1.alloc(m->len1 * 4)) || (rc = m->cnt2.alloc(m->len2 * 4)) ||
      (rc = m->acc1.alloc(m->len1 * 8)) || (rc = m->acc2.alloc(m->len2 * 8))) {
    delete m;
    return rc;
  }
  hipError_t e = hipStreamSynchronize(p->ctx->stream);  // uploads read host vectors
  if (e != hipSuccess) {
    delete m;
    return hip_fail(e, "moment spec upload");
  }
  *out = m;
  return THRML_OK;
}

extern "C" void thrml_moments_destroy(thrml_moments *m) {
  if (!m) return;
  (void)hipSetDevice(m->ctx->device);
  (void)hipStreamSynchronize(m->ctx->stream);
  delete m;
}

extern "C" int thrml_moments_run(thrml_prog *p, uint64_t key, thrml_schedule sched,
                                 thrml_state *st, thrml_moments *m, int64_t *node_sums,
                                 int64_t *pair_sums, int out_on_device) {
  if (!p || !st || !m) return fail(THRML_EINVAL, "NULL argument");
  if (st->prog != p) return fail(THRML_EINVAL, "state belongs to another program");
  if (m->prog != p) return fail(THRML_EINVAL, "moment spec belongs to another program");
  if ((m->n1 && !node_sums) || (m->n2 && !pair_sums)) return fail(THRML_EINVAL, "NULL argument");
  THRML_HIP(hipSetDevice(p->ctx->device));
  if (int rc = not_observing(p->ctx)) return rc;
  std::lock_guard<std::mutex> lk(p->ctx->run_mu);
  hipStream_t s = p->ctx->stream;
  THRML_HIP(hipMemsetAsync(m->cnt1.p, 0, m->cnt1.bytes, s));
  THRML_HIP(hipMemsetAsync(m->cnt2.p, 0, m->cnt2.bytes, s));
  THRML_HIP(hipMemsetAsync(m->acc1.p, 0, m->acc1.bytes, s));
  THRML_HIP(hipMemsetAsync(m->acc2.p, 0, m->acc2.bytes, s));
  uint32_t *c1 = m->cnt1.as<uint32_t>(), *c2 = m->cnt2.as<uint32_t>();
  uint64_t n_obs = 0, since_fold = 0;
  const uint64_t max_before_fold = 0xffffffffull / st->C;  // counters grow <= C per observation
  LatticeMoments lm{c1, c2};
  auto obs = [&](bool fused) -> int {
    if (!fused) {
      const int r = m->native ? launch_lattice_moments(st, &lm)
                              : launch_moments(st, m->npos.as<uint32_t>(), m->n1,
                                               m->ppos.as<uint32_t>(), m->n2, c1, c2);
      if (r) return r;
    }
    ++n_obs;
    if (++since_fold >= max_before_fold) {
      since_fold = 0;
      if (int r = launch_fold_counts(p->ctx, c1, m->acc1.as<uint64_t>(), m->len1)) return r;
      return launch_fold_counts(p->ctx, c2, m->acc2.as<uint64_t>(), m->len2);
    }
    return THRML_OK;
  };
  KeyStore ks;
  ks.grow = &p->ctx->keys;
  int rc = run_plan(p, st, schedule_plan(p, st, key, sched), m->native ? &lm : nullptr, obs, ks);
  if (rc) return rc;
  int64_t *o1 = node_sums, *o2 = pair_sums;
  if (!out_on_device) {
    if ((rc = m->out.alloc((m->n1 + m->n2) * 8))) return rc;
    o1 = m->out.as<int64_t>();
    o2 = o1 + m->n1;
  }
  const int64_t cn = (int64_t)st->C * (int64_t)n_obs;
  rc = launch_finalize_moments(p->ctx, c1, m->acc1.as<uint64_t>(),
                               m->native ? m->slot1.as<uint32_t>() : nullptr, m->n1, c2,
                               m->acc2.as<uint64_t>(), m->native ? m->slot2.as<uint32_t>() : nullptr,
                               m->n2, cn, o1, o2);
  if (rc) return rc;
  if (!out_on_device) {
    if (m->n1) THRML_HIP(hipMemcpyAsync(node_sums, o1, m->n1 * 8, hipMemcpyDeviceToHost, s));
    if (m->n2) THRML_HIP(hipMemcpyAsync(pair_sums, o2, m->n2 * 8, hipMemcpyDeviceToHost, s));
    THRML_HIP(hipStreamSynchronize(s));
  }
  return THRML_OK;
}

extern "C" int thrml_observer_create(thrml_prog *p, const uint64_t *row_offsets, uint64_t n_rows,
                                     const uint32_t *nodes, int transform_to_spin,
                                     thrml_observer **out) {
  if (!p || !out || (n_rows && !row_offsets)) return fail(THRML_EINVAL, "NULL argument");
  if (n_rows && row_offsets[0] != 0) return fail(THRML_EINVAL, "row offsets must start at 0");
  for (uint64_t r = 0; r < n_rows; ++r)
    if (row_offsets[r + 1] < row_offsets[r]) return fail(THRML_EINVAL, "row offsets must not decrease");
  const uint64_t n_nodes = n_rows ? row_offsets[n_rows] : 0;
  if (n_nodes && !nodes) return fail(THRML_EINVAL, "NULL argument");
  std::vector<uint32_t> pos(n_nodes + 1, 0u);
  for (uint64_t k = 0; k < n_nodes; ++k) {
    if (nodes[k] >= p->node_pos.size() || p->node_pos[nodes[k]] < 0)
      return fail(THRML_EINVAL, "Node not found in global location map");
    pos[k] = (uint32_t)p->node_pos[nodes[k]];
  }
  // Byte states multiply category values in int64: each row's product must
  // fit, whatever the values (|2x - 1| <= 2q - 3, or x <= q - 1)
  double max_log2 = 0.0;
  if (byte_layout(p)) {
    for (uint64_t r = 0; r < n_rows; ++r) {
      double l = 0.0;
      for (uint64_t k = row_offsets[r]; k < row_offsets[r + 1]; ++k) {
        const uint32_t b = (uint32_t)(std::upper_bound(p->blk_off.begin(), p->blk_off.end(),
                                                       (uint64_t)pos[k]) - p->blk_off.begin() - 1);
        const uint32_t q = block_q(p, std::min(b, p->n_free + p->n_clamped - 1));
        const double m = transform_to_spin ? 2.0 * q - 3.0 : q - 1.0;
        if (m > 1.0) l += std::log2(m);
      }
      if (l > 62.0)
        return fail(THRML_EINVAL, "moment row " + std::to_string(r) +
                                      ": its product of category values can exceed int64");
      max_log2 = std::max(max_log2, l);
    }
  }
  THRML_HIP(hipSetDevice(p->ctx->device));
  auto *o = new thrml_observer();
  o->prog = p;
  o->ctx = p->ctx;
  o->n_rows = n_rows;
  o->transform = transform_to_spin != 0;
  o->max_row_log2 = max_log2;
  std::vector<uint64_t> off(row_offsets, row_offsets + n_rows + (n_rows ? 1 : 0));
  if (off.empty()) off.push_back(0);
  int rc = upload_to(p->ctx, o->row_off, off);
  if (!rc) rc = upload_to(p->ctx, o->pos, pos);
  if (!rc) rc = o->acc.alloc(std::max<uint64_t>(n_rows, 1) * sizeof(int64_t));
  if (!rc) {
    hipError_t e = hipStreamSynchronize(p->ctx->stream);
    if (e != hipSuccess) rc = hip_fail(e, "observer upload");
  }
  if (rc) {
    delete o;
    return rc;
  }
  *out = o;
  return THRML_OK;
}

extern "C" void thrml_observer_destroy(thrml_observer *o) {
  if (!o) return;
  (void)hipSetDevice(o->ctx->device);
  (void)hipStreamSynchronize(o->ctx->stream);
  delete o;
}

extern "C" int thrml_observer_run(thrml_prog *p, uint64_t key, thrml_schedule sched,
                                  thrml_state *st, thrml_observer *o, int64_t *sums,
                                  int sums_on_device) {
  if (!p || !st || !o || (o->n_rows && !sums)) return fail(THRML_EINVAL, "NULL argument");
  if (st->prog != p) return fail(THRML_EINVAL, "state belongs to another program");
  if (o->prog != p) return fail(THRML_EINVAL, "observer belongs to another program");
  if (o->max_row_log2 > 0.0 &&
      o->max_row_log2 + std::log2((double)st->C) +
              std::log2((double)std::max<uint64_t>(sched.n_samples, 1)) >= 63.0)
    return fail(THRML_EINVAL, "the moment sums of this run (chains x observations x the largest "
                              "product of category values) can exceed int64");
  THRML_HIP(hipSetDevice(p->ctx->device));
  if (int rc = not_observing(p->ctx)) return rc;
  std::lock_guard<std::mutex> lk(p->ctx->run_mu);
  hipStream_t s = p->ctx->stream;
  THRML_HIP(hipMemsetAsync(o->acc.p, 0, o->acc.bytes, s));
  auto obs = [&](bool) -> int { return launch_observe(st, o); };
  KeyStore ks;
  ks.grow = &p->ctx->keys;
  if (int rc = run_plan(p, st, schedule_plan(p, st, key, sched), nullptr, obs, ks)) return rc;
  if (o->n_rows) {
    const size_t bytes = o->n_rows * sizeof(int64_t);
    THRML_HIP(hipMemcpyAsync(sums, o->acc.p, bytes,
                             sums_on_device ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost, s));
  }
  if (!sums_on_device) THRML_HIP(hipStreamSynchronize(s));
  return THRML_OK;
}

extern "C" int thrml_estimate_moments(thrml_prog *p, uint64_t key, thrml_schedule sched,
                                      thrml_state *st, const uint32_t *nodes, uint64_t n1,
                                      const uint32_t *pairs, uint64_t n2, int64_t *node_sums,
                                      int64_t *pair_sums) {
  if (!p || !st) return fail(THRML_EINVAL, "NULL argument");
  if (st->prog != p) return fail(THRML_EINVAL, "state belongs to another program");
  if ((n1 && !node_sums) || (n2 && !pair_sums)) return fail(THRML_EINVAL, "NULL argument");
  thrml_moments *m = nullptr;
  if (int rc = thrml_moments_create(p, nodes, n1, pairs, n2, &m)) return rc;
  const int rc = thrml_moments_run(p, key, sched, st, m, node_sums, pair_sums, 0);
  thrml_moments_destroy(m);
  return rc;
}

extern "C" int thrml_sample_with_observer(thrml_prog *p, uint64_t key, thrml_schedule sched,
                                          thrml_state *st, thrml_observe_fn observe, void *user) {
  if (!p || !st || !observe) return fail(THRML_EINVAL, "NULL argument");
  if (st->prog != p) return fail(THRML_EINVAL, "state belongs to another program");
  if (int rc = not_observing(p->ctx)) return rc;
  THRML_HIP(hipSetDevice(p->ctx->device));
  std::lock_guard<std::mutex> lk(p->ctx->run_mu);
  uint64_t iteration = 0;
  auto obs = [&](bool) -> int {
    int rc;
    {
      ObservingScope scope(p->ctx);
      rc = observe(user, iteration++, st, reinterpret_cast<void *>(p->ctx->stream));
    }
    if (rc) return fail(rc, "the observer callback returned " + std::to_string(rc) +
                                " at iteration " + std::to_string(iteration - 1));
    return THRML_OK;
  };
  KeyStore ks;
  ks.grow = &p->ctx->keys;
  return run_plan(p, st, schedule_plan(p, st, key, sched), nullptr, obs, ks);
}

extern "C" int thrml_sample_states_as(thrml_prog *p, uint64_t key, thrml_schedule sched,
                                      thrml_state *st, void *out, int dtype) {
  if (!p || !st || !out) return fail(THRML_EINVAL, "NULL argument");
  if (st->prog != p) return fail(THRML_EINVAL, "state belongs to another program");
  if (dtype != THRML_DTYPE_U8 && dtype != THRML_DTYPE_F32) return fail(THRML_EINVAL, "unknown dtype");
  if (dtype == THRML_DTYPE_U8 && p->cat_bytes == 2)
    return fail(THRML_EINVAL, "categories above 255 do not fit the u8 dtype: sample this program's "
                              "states as f32");
  THRML_HIP(hipSetDevice(p->ctx->device));
  const uint32_t nb = p->n_free + p->n_clamped;
  const size_t esz = dtype == THRML_DTYPE_U8 ? 1 : 4;
  const size_t per = (size_t)st->C * p->n_total * esz;  // bytes of one observation
  DevBuf tmp;
  if (int rc = tmp.alloc(per)) return rc;
  std::vector<uint8_t> blk;
  uint64_t k_obs = 0;
  auto obs = [&](bool) -> int {
    uint8_t *dst = static_cast<uint8_t *>(out) + k_obs * per;
    for (uint32_t b = 0; b < nb; ++b) {
      const size_t n_b = p->blk_off[b + 1] - p->blk_off[b];
      uint8_t *dblk = tmp.as<uint8_t>() + (size_t)st->C * p->blk_off[b] * esz;
      const int rc = byte_layout(p) ? launch_potts_unpack(st, b, dblk, dtype)
                                        : launch_unpack(st, b, dblk, dtype);
      if (rc) return rc;
      blk.resize((size_t)st->C * n_b * esz);
      THRML_HIP(hipMemcpyAsync(blk.data(), dblk, blk.size(), hipMemcpyDeviceToHost, p->ctx->stream));
      THRML_HIP(hipStreamSynchronize(p->ctx->stream));
      for (uint32_t c = 0; c < st->C; ++c)
        std::memcpy(dst + ((size_t)c * p->n_total + p->blk_off[b]) * esz,
                    blk.data() + (size_t)c * n_b * esz, n_b * esz);
    }
    ++k_obs;
    return THRML_OK;
  };
  if (int rc = not_observing(p->ctx)) return rc;
  std::lock_guard<std::mutex> lk(p->ctx->run_mu);
  KeyStore ks;
  ks.grow = &p->ctx->keys;
  return run_plan(p, st, schedule_plan(p, st, key, sched), nullptr, obs, ks);
}

extern "C" int thrml_sample_states(thrml_prog *p, uint64_t key, thrml_schedule sched,
                                   thrml_state *st, uint8_t *out) {
  return thrml_sample_states_as(p, key, sched, st, out, THRML_DTYPE_U8);
}

extern "C" int thrml_hinton_init(thrml_prog *p, uint64_t key, thrml_state *st) {
  if (!p || !st) return fail(THRML_EINVAL, "NULL argument");
  if (st->prog != p) return fail(THRML_EINVAL, "state belongs to another program");
  if (int rc = not_observing(p->ctx)) return rc;
  if (byte_layout(p)) return fail(THRML_EINVAL, "hinton_init is defined for Ising programs");
  THRML_HIP(hipSetDevice(p->ctx->device));
  std::vector<uint64_t> bk(p->n_free);
  thrml_rng_split(key, p->n_free, bk.data());
  const uint64_t nf = p->blk_off[p->n_free];
  std::vector<float> prob(nf);
  for (uint64_t k = 0; k < nf; ++k) prob[k] = sigmoid_b(p->bias_raw[p->pos_node[k]] * p->beta);  // ising.rs:650
  std::vector<uint32_t> k8(8 * p->n_free);
  for (uint32_t b = 0; b < p->n_free; ++b) {
    const Key8 e = seed_from_u64(bk[b]);
    for (int i = 0; i < 8; ++i) k8[8 * b + i] = e.k[i];
  }
  DevBuf dk, dp;
  int rc;
  if ((rc = dk.alloc(k8.size() * 4)) || (rc = dp.alloc(prob.size() * 4))) return rc;
  THRML_HIP(hipMemcpyAsync(dk.p, k8.data(), k8.size() * 4, hipMemcpyHostToDevice, p->ctx->stream));
  THRML_HIP(hipMemcpyAsync(dp.p, prob.data(), prob.size() * 4, hipMemcpyHostToDevice, p->ctx->stream));
  for (uint32_t b = 0; b < p->n_free; ++b) {
    if ((rc = launch_hinton(p, st, b, dk.as<uint32_t>() + 8 * b, dp.as<float>() + p->blk_off[b]))) return rc;
  }
  if (p->kind == K_DENSE)
    for (uint32_t b = 0; b < 2; ++b)
      if ((rc = launch_dense_sync_act(st, b))) return rc;
  THRML_HIP(hipStreamSynchronize(p->ctx->stream));
  return THRML_OK;
}

extern "C" int thrml_ising_energy(thrml_prog *p, thrml_state *st, double *out) {
  if (!p || !st || !out) return fail(THRML_EINVAL, "NULL argument");
  if (st->prog != p) return fail(THRML_EINVAL, "state belongs to another program");
  if (p->kind == K_POTTS) return fail(THRML_EINVAL, "not a spin program (use thrml_potts_energy)");
  if (p->kind == K_DISCRETE) return fail(THRML_EINVAL, "not an Ising program (use thrml_discrete_energy)");
  THRML_HIP(hipSetDevice(p->ctx->device));
  return spin_energy(p, st, out);
}

extern "C" int thrml_potts_energy(thrml_prog *p, thrml_state *st, double *out) {
  if (!p || !st || !out) return fail(THRML_EINVAL, "NULL argument");
  if (st->prog != p) return fail(THRML_EINVAL, "state belongs to another program");
  if (p->kind != K_POTTS) return fail(THRML_EINVAL, "not a categorical program");
  THRML_HIP(hipSetDevice(p->ctx->device));
  return potts_energy(p, st, out);
}

extern "C" int thrml_discrete_energy(thrml_prog *p, thrml_state *st, double *out) {
  if (!p || !st || !out) return fail(THRML_EINVAL, "NULL argument");
  if (st->prog != p) return fail(THRML_EINVAL, "state belongs to another program");
  if (p->kind != K_DISCRETE) return fail(THRML_EINVAL, "not a discrete factor program");
  THRML_HIP(hipSetDevice(p->ctx->device));
  return discrete_energy(p, st, out);
}

extern "C" int thrml_sigmoid_bernoulli(thrml_ctx *ctx, const float *g, const float *u, float *o,
                                       uint64_t n) {
  if (!ctx || (n && (!g || !u || !o))) return fail(THRML_EINVAL, "NULL argument");
  THRML_HIP(hipSetDevice(ctx->device));
  return launch_sigmoid_bernoulli(ctx, g, u, o, n);
}

extern "C" int thrml_gumbel_argmax(thrml_ctx *ctx, const float *l, const float *u, int32_t *o,
                                   uint64_t n, uint32_t q) {
  if (!ctx || (n && (!l || !u || !o))) return fail(THRML_EINVAL, "NULL argument");
  if (q == 0) return fail(THRML_EINVAL, "q must be positive");
  THRML_HIP(hipSetDevice(ctx->device));
  return launch_gumbel_argmax(ctx, l, u, o, n, q);
}

extern "C" int thrml_batch_gather(thrml_ctx *ctx, const float *weights, uint64_t n_weights,
                                  const int32_t *indices, uint64_t batch, uint32_t n_indices,
                                  const uint32_t *strides, uint32_t batch_stride, float *out) {
  if (!ctx || (batch && (!weights || !out || (n_indices && (!indices || !strides)))))
    return fail(THRML_EINVAL, "NULL argument");
  if (n_indices > BATCH_GATHER_MAX_INDICES)
    return fail(THRML_EUNSUPPORTED, "at most " + std::to_string(BATCH_GATHER_MAX_INDICES) +
                                        " indices per batch element");
  if (batch > 0xffffffffull) return fail(THRML_EINVAL, "batch must stay below 2^32");
  BatchGatherStrides st{};
  for (uint32_t i = 0; i < n_indices; ++i) st.s[i] = strides[i];
  st.batch_stride = batch_stride;
  THRML_HIP(hipSetDevice(ctx->device));
  return launch_batch_gather(ctx, weights, n_weights, indices, batch, n_indices, st, out);
}

extern "C" int thrml_fast_math_check(thrml_ctx *ctx, float *out) {
  if (!ctx || !out) return fail(THRML_EINVAL, "NULL argument");
  THRML_HIP(hipSetDevice(ctx->device));
  return launch_fast_math_check(ctx, out);
}

extern "C" int thrml_fast_math_status(thrml_ctx *ctx, float *out, int *ok) {
  if (!ctx || !out || !ok) return fail(THRML_EINVAL, "NULL argument");
  THRML_HIP(hipSetDevice(ctx->device));
  return fast_math_gate(ctx, out, ok);
}
