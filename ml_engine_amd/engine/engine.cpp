// Runtime, memory, NodeBackProp, AdamParameter, dispatch (GraphOperations
// forward / backward / zero_grad / ParameterUpdate / accumulate / clipNorm),
// Linear, Convolute2D and Embedding.  Reference: Engine/engine.cu:1-330,
// 652-673, 3349-3606, 3723-3817; Engine/transformer.cu:176-245.
#include "engine.h"

#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <map>
#include <mutex>
#include <random>
#include <unordered_set>

namespace mle {

// ---------------------------------------------------------------------------
// stream and errors
static mle_stream g_stream = nullptr;
static bool g_stream_made = false;

void check(int rc, const str& what) {
  if (rc != MLE_OK) {
    std::cerr << what << ": " << mle_last_error() << std::endl;
    std::exit(1);
  }
}

mle_stream stream() {
  if (!g_stream_made) {
    check(mle_init(0), "mle_init");
    check(mle_stream_create(&g_stream), "stream create");
    g_stream_made = true;
  }
  return g_stream;
}

void set_stream(mle_stream s) {
  g_stream = s;
  g_stream_made = true;
}

void sync(const str& what) { check(mle_stream_sync(stream()), what); }

// ---------------------------------------------------------------------------
// chunked device arenas with exact-size reuse
namespace {
struct Arena {
  std::vector<std::pair<char*, size_t>> chunks;  // base, capacity
  size_t used = 0;                               // in the last chunk
  std::multimap<size_t, char*> free_blocks;      // size -> block
  size_t chunk_bytes = size_t(1) << 30;

  char* take(size_t bytes) {
    bytes = (bytes + 255) & ~size_t(255);
    if (bytes == 0) bytes = 256;
    auto it = free_blocks.find(bytes);
    if (it != free_blocks.end()) {
      char* p = it->second;
      free_blocks.erase(it);
      return p;
    }
    if (chunks.empty() || used + bytes > chunks.back().second) {
      const size_t cap = std::max(chunk_bytes, bytes);
      void* p = nullptr;
      check(mle_device_alloc(&p, cap), "SafeCudaMalloc (arena chunk)");
      chunks.push_back({static_cast<char*>(p), cap});
      used = 0;
    }
    char* p = chunks.back().first + used;
    used += bytes;
    return p;
  }
  void give(char* p, size_t bytes) {
    bytes = (bytes + 255) & ~size_t(255);
    if (bytes == 0) bytes = 256;
    free_blocks.insert({bytes, p});
  }
};
Arena g_out, g_grad, g_scratch;
std::mutex g_mem_mu;
}  // namespace

float* alloc_output(size_t n) {
  std::lock_guard<std::mutex> lk(g_mem_mu);
  return reinterpret_cast<float*>(g_out.take(n * sizeof(float)));
}
float* alloc_grad(size_t n) {
  std::lock_guard<std::mutex> lk(g_mem_mu);
  return reinterpret_cast<float*>(g_grad.take(n * sizeof(float)));
}
void release(float* p, size_t n, bool grad) {
  if (!p) return;
  std::lock_guard<std::mutex> lk(g_mem_mu);
  (grad ? g_grad : g_out).give(reinterpret_cast<char*>(p), n * sizeof(float));
}
void* alloc_scratch(size_t bytes) {
  std::lock_guard<std::mutex> lk(g_mem_mu);
  return g_scratch.take(bytes);
}

void* gemm_workspace(size_t bytes) {
  static void* ws = nullptr;
  static size_t cap = 0;
  if (bytes == 0) return ws;
  if (bytes > cap) {
    ws = alloc_scratch(bytes);
    cap = bytes;
  }
  return ws;
}

// ---------------------------------------------------------------------------
// batched zeroing
namespace {
int g_zero_depth = 0;
std::vector<std::pair<float*, size_t>> g_zero_ranges;
}  // namespace

void zero(float* p, size_t n) {
  if (!p || n == 0) return;
  if (g_zero_depth > 0) {
    g_zero_ranges.push_back({p, n});
    return;
  }
  check(mle_fill(stream(), p, 0.0f, n), "Zero_grad");
}

ZeroBatch::ZeroBatch() { ++g_zero_depth; }
ZeroBatch::~ZeroBatch() {
  if (--g_zero_depth > 0) return;
  auto r = std::move(g_zero_ranges);
  g_zero_ranges.clear();
  std::sort(r.begin(), r.end());
  // Every tensor starts on a 256-byte boundary and owns the padding up to the
  // next one, so a range may be merged with the next when that one starts
  // inside its padded extent; the padding cleared in between belongs to no
  // other tensor.
  auto padded_end = [](const std::pair<float*, size_t>& x) { return x.first + ((x.second + 63) & ~size_t(63)); };
  size_t i = 0;
  while (i < r.size()) {
    float* b = r[i].first;
    float* e = r[i].first + r[i].second;
    float* ep = padded_end(r[i]);
    size_t j = i + 1;
    while (j < r.size() && r[j].first <= ep) {
      e = std::max(e, r[j].first + r[j].second);
      ep = std::max(ep, padded_end(r[j]));
      ++j;
    }
    check(mle_fill(stream(), b, 0.0f, (size_t)(e - b)), "Zero_grad");
    i = j;
  }
}

static bool g_lazy_zero = true;
void set_lazy_zero(bool on) { g_lazy_zero = on; }

void defer_zero(NodeBackProp* n) {
  if (!n || !n->grad || n->total <= 0) return;
  n->grad_src = nullptr;
  n->grad_early = false;
  if (g_lazy_zero) n->grad_pending_zero = true;
  else zero(n->grad, n->total);
}

int accumulate_flag(NodeBackProp* n) {
  resolve_alias(n);
  if (n->grad_pending_zero) {
    n->grad_pending_zero = false;
    n->grad_early = false;  // the caller writes the whole gradient
    return 0;
  }
  return 1;
}

const float* grad_of(const NodeBackProp* n) { return n->grad_src ? n->grad_src : n->grad; }

bool can_alias_grad(const NodeBackProp* in, const NodeBackProp* from) {
  if (!g_lazy_zero || !fusion_enabled() || !in || !from || in == from || !in->reads_grad_alias) return false;
  if (!in->grad_pending_zero || in->grad_src || in->total != from->total) return false;
  if (in->consumers == 1) return true;
  // One other consumer still to come, which may be a normalisation whose
  // second pass adds into this node's gradient at this node's place: it reads
  // the alias where a copy would be written (norm_node); any other consumer
  // resolves the alias before it adds (accumulate_flag).
  return in->takes_norm_grad && in->consumers == 2 && in->consumers_done == 0;
}

bool alias_grad(NodeBackProp* in, const NodeBackProp* from) {
  if (!can_alias_grad(in, from)) return false;
  in->grad_src = grad_of(from);
  in->grad_pending_zero = false;  // its gradient is defined: the alias's content
  return true;
}

void resolve_alias(NodeBackProp* n) {
  if (!n || !n->grad_src) return;
  const float* src = n->grad_src;
  n->grad_src = nullptr;
  check(mle_scale_assign(stream(), src, n->grad, 1.0, n->total), "gradient of " + n->op_name);
}

int params_write_flag(const std::vector<NodeBackProp*>& ps) {
  bool all = true;
  for (auto* p : ps)
    if (p) all = all && p->grad_pending_zero;
  if (all) {
    for (auto* p : ps)
      if (p) p->grad_pending_zero = false;
    return 0;
  }
  for (auto* p : ps)
    if (p) materialize(p);
  return 1;
}

void materialize_params(const std::vector<AdamParameter*>& ps) {
  // Fills only: a pending clip stays deferred (the fused update divides in
  // registers; the other callers apply the clip themselves first).
  ZeroBatch batch;  // neighbouring parameters' fills merge into one launch
  for (auto* p : ps)
    if (p->grad_pending_zero) {
      p->grad_pending_zero = false;
      zero(p->grad, p->total);
    }
}

void materialize(NodeBackProp* n) {
  if (!n) return;
  resolve_alias(n);
  clip_apply(n);
  if (!n->grad_pending_zero) return;
  n->grad_pending_zero = false;
  n->grad_early = false;
  zero(n->grad, n->total);
}

void defer_zero_output(NodeBackProp* n) {
  if (!n || !n->output || n->total <= 0) return;
  if (g_lazy_zero) n->output_pending_zero = true;
  else zero(n->output, n->total);
}

void materialize_output(NodeBackProp* n) {
  if (!n) return;
  // Kept for the next read: graph replays run no host code to mark the
  // output stale again, and the refresh leaves a current output unchanged.
  if (n->output_refresh) n->output_refresh();
  if (!n->output_pending_zero) return;
  n->output_pending_zero = false;
  zero(n->output, n->total);
}

// ---------------------------------------------------------------------------
// pending global-norm clip
namespace {
double* g_clip_snapshot = nullptr;             // device double: s as clipNorm saw it
std::unordered_set<NodeBackProp*> g_clip_marked;  // parameters whose gradient reads as g / s
}  // namespace

void clip_mark(const std::vector<AdamParameter*>& ps, const double* s) {
  clip_apply_all();
  materialize_params(ps);  // a marked gradient is divided in place later
  if (!g_clip_snapshot) g_clip_snapshot = static_cast<double*>(alloc_scratch(256));
  check(mle_memcpy_d2d(g_clip_snapshot, s, sizeof(double), stream()), "clipNorm: snapshot of the scale");
  for (auto* p : ps) g_clip_marked.insert(p);
}

const double* clip_view(const std::vector<AdamParameter*>& ps) {
  if (g_clip_marked.empty()) return nullptr;
  bool all = g_clip_marked.size() == ps.size();
  for (auto* p : ps) all = all && g_clip_marked.count(p);
  if (all) return g_clip_snapshot;
  clip_apply_all();
  return nullptr;
}

void clip_apply(NodeBackProp* p) {
  if (g_clip_marked.empty() || !g_clip_marked.erase(p)) return;
  check(mle_scale_by_device(stream(), p->grad, g_clip_snapshot, 1, p->total), "ScalePtr of " + p->op_name);
}

void clip_apply_all() {
  auto marked = std::move(g_clip_marked);
  g_clip_marked.clear();
  for (auto* p : marked)
    check(mle_scale_by_device(stream(), p->grad, g_clip_snapshot, 1, p->total), "ScalePtr of " + p->op_name);
}

void clip_drop(NodeBackProp* p) { g_clip_marked.erase(p); }

void clip_clear() { g_clip_marked.clear(); }

size_t clip_marked_count() { return g_clip_marked.size(); }

// ---------------------------------------------------------------------------
// flat parameter arena
namespace {
struct Slab {
  float* base;
  size_t cap;
  size_t used;
};
std::vector<Slab> g_slabs;
size_t g_next_slab = size_t(64) << 20;
uint64_t g_seed = 0;
bool g_seed_set = false;

bool g_open_new_slab = false;
}  // namespace

// The next `floats` of parameters are meant to be contiguous: if the current
// slab cannot hold them all, the next allocation opens a slab that can.
void param_reserve(size_t floats) {
  g_next_slab = std::max<size_t>(floats, 64);
  g_open_new_slab = g_slabs.empty() || g_slabs.back().used + floats > g_slabs.back().cap;
}

ParamSlot param_alloc(size_t n, float** p, float** g, float** m, float** v) {
  const size_t need = (n + 63) & ~size_t(63);
  if (g_slabs.empty() || g_open_new_slab || g_slabs.back().used + need > g_slabs.back().cap) {
    g_open_new_slab = false;
    const size_t cap = std::max(g_next_slab, need);
    void* base = nullptr;
    check(mle_device_alloc(&base, cap * 4 * sizeof(float)), "SafeCudaMalloc (parameter arena)");
    // Zero all four regions once: the padding between parameters must read as
    // 0 when the optimizer and the norm sweep a contiguous span.
    check(mle_fill(stream(), static_cast<float*>(base), 0.0f, cap * 4), "parameter arena clear");
    g_slabs.push_back({static_cast<float*>(base), cap, 0});
  }
  Slab& s = g_slabs.back();
  const size_t off = s.used;
  s.used += need;
  *p = s.base + off;
  *g = s.base + s.cap + off;
  *m = s.base + 2 * s.cap + off;
  *v = s.base + 3 * s.cap + off;
  return ParamSlot{(int)g_slabs.size() - 1, off};
}

void set_init_seed(uint64_t seed) {
  g_seed = seed;
  g_seed_set = true;
}

static uint64_t next_seed() {
  if (g_seed_set) return g_seed++;
  std::random_device rd;
  return ((uint64_t)rd() << 32) | rd();
}

Quirks& quirks() {
  static Quirks q;
  return q;
}

}  // namespace mle

using mle::check;

// ---------------------------------------------------------------------------
// NodeBackProp (Engine/engine.cu:45-124)
NodeBackProp::NodeBackProp(str name, int batch, int d1, int d2, int d3, int allocation) : op_name(name) {
  dim[0] = batch;
  dim[1] = d1;
  dim[2] = d2;
  dim[3] = d3;
  total = (long long)batch * d1 * d2 * d3;
  if (allocation == 1) {
    output = mle::alloc_output(total);
    grad = mle::alloc_grad(total);
    check(mle_fill(mle::stream(), grad, 0.0f, total), "Fill Kernel for Gradient");
    owns_ = true;
  }
}

void NodeBackProp::clear() {
  if (owns_) {
    mle::release(output, total, false);
    mle::release(grad, total, true);
    owns_ = false;
  }
  output = grad = nullptr;
  inputs.clear();
  op_name.clear();
}

static void reshape_check(NodeBackProp* n, const int* d, int size) {
  if (size != 4) {
    std::cerr << "Reshape only supports 4D tensors\n";
    std::exit(1);
  }
  const long long nt = (long long)d[0] * d[1] * d[2] * d[3];
  if (nt != n->total) {
    std::cerr << "Reshape cannot change total size of tensor\n";
    std::cout << "Dimensions for node: " << n->op_name << "\n";
    std::exit(1);
  }
  for (int i = 0; i < 4; ++i) n->dim[i] = d[i];
}
void NodeBackProp::reshape(std::vector<int> nd) { reshape_check(this, nd.data(), (int)nd.size()); }
void NodeBackProp::reshape(int arr[], const int size) { reshape_check(this, arr, size); }

void CheckError(const str& reason) {
  const int rc = mle_stream_sync(mle::stream());
  if (rc != MLE_OK) {
    std::cerr << "Runtime error in " << reason << ": " << mle_last_error() << std::endl;
    std::exit(1);
  }
}

float ReadValueAt(const graph& X, const int& idx, const bool g) {
  if (g) mle::materialize(X.get());
  else mle::materialize_output(X.get());
  float out = 0.f;
  check(mle_memcpy_d2h(&out, (g ? X->grad : X->output) + idx, sizeof(float), mle::stream()), "ReadValueAt");
  return out;
}

void WriteValueAt(const graph& X, const float value, const int& idx, const bool g) {
  if (g) mle::materialize(X.get());
  else mle::materialize_output(X.get());
  check(mle_memcpy_h2d((g ? X->grad : X->output) + idx, &value, sizeof(float), mle::stream()), "WriteValueAt");
}

// ---------------------------------------------------------------------------
// AdamParameter (Engine/engine.cu:126-302)
AdamParameter::AdamParameter(str n, int out, int in, int row, int col, double norm)
    : NodeBackProp(n, out, in, row, col, 0),
      t(1),
      b1(0.9f),
      b2(0.999f),
      epsilon(1e-8f),
      batch_size(0),
      group_norm((float)norm),
      weight_decay(0.01f) {
  slot = mle::param_alloc(total, &output, &grad, &m, &v);
  // Standard_Weights: U(-1, 1) * sqrt(XAVIER / (in*row*col)) (Engine/kernels.cu:953-960),
  // drawn on the host from a seeded engine (the reference draws curand Philox
  // seeded from std::random_device).
  std::mt19937_64 gen(mle::next_seed());
  std::uniform_real_distribution<float> dist(-1.0f, 1.0f);
  const float scale = sqrtf(XAVIER / (float)((long long)in * row * col));
  std::vector<float> host(total);
  for (auto& x : host) x = dist(gen) * scale;
  check(mle_memcpy_h2d(output, host.data(), total * sizeof(float), mle::stream()), "AdamParameter init");
  check(mle_fill(mle::stream(), grad, 0.0f, total), "AdamParameter grad");
  check(mle_fill(mle::stream(), m, 0.0f, total), "AdamParameter m");
  check(mle_fill(mle::stream(), v, 0.0f, total), "AdamParameter v");
}

AdamParameter::~AdamParameter() { mle::clip_drop(this); }

// File layout: [u32 name_len][name][i32 total][f32 W * total][f32 m * total][f32 v * total]
// (Engine/engine.cu:139-184); `t` is not stored, as in the reference.
void AdamParameter::save(std::ofstream& f) const {
  const uint32_t name_len = (uint32_t)op_name.size();
  f.write(reinterpret_cast<const char*>(&name_len), sizeof(uint32_t));
  f.write(op_name.data(), name_len);
  const int tot = (int)total;
  f.write(reinterpret_cast<const char*>(&tot), sizeof(int));
  if (!f) {
    std::cerr << "File write failed saving parameter header: " << op_name << "\n";
    std::exit(1);
  }
  std::vector<float> host(total);
  const float* src[3] = {output, m, v};
  for (int i = 0; i < 3; ++i) {
    check(mle_memcpy_d2h(host.data(), src[i], total * sizeof(float), mle::stream()), "save " + op_name);
    f.write(reinterpret_cast<const char*>(host.data()), total * sizeof(float));
    if (!f) {
      std::cerr << "File write failed saving " << op_name << "\n";
      std::exit(1);
    }
  }
}

void AdamParameter::load(std::ifstream& f) {
  uint32_t name_len = 0;
  f.read(reinterpret_cast<char*>(&name_len), sizeof(uint32_t));
  if (!f) {
    std::cerr << "File read failed reading name length for: " << op_name << "\n";
    std::exit(1);
  }
  std::string loaded(name_len, '\0');
  f.read(&loaded[0], name_len);
  if (!f) {
    std::cerr << "File read failed reading name for: " << op_name << "\n";
    std::exit(1);
  }
  if (loaded != op_name) {
    std::cerr << "Parameter name mismatch: expected '" << op_name << "' but got '" << loaded << "'\n";
    std::exit(1);
  }
  int tot = 0;
  f.read(reinterpret_cast<char*>(&tot), sizeof(int));
  if (!f) {
    std::cerr << "File read failed reading size for: " << op_name << "\n";
    std::exit(1);
  }
  if (tot != total) {
    std::cerr << "Parameter size mismatch for '" << op_name << "': expected " << total << " but loaded " << tot << "\n";
    std::exit(1);
  }
  std::vector<float> host(total);
  float* dst[3] = {output, m, v};
  for (int i = 0; i < 3; ++i) {
    f.read(reinterpret_cast<char*>(host.data()), total * sizeof(float));
    if (!f) {
      std::cerr << "File read failed loading " << op_name << "\n";
      std::exit(1);
    }
    check(mle_memcpy_h2d(dst[i], host.data(), total * sizeof(float), mle::stream()), "load " + op_name);
  }
}

void AdamParameter::update(const float lr, const bool W) {
  mle::materialize(this);
  check(mle_adam_update(mle::stream(), output, grad, m, v, total, t, lr, b1, b2, epsilon, weight_decay, W ? 1 : 0,
                        nullptr),
        "AdamUpdate in AdamParameter update");
  t++;
}

void AdamParameter::accumulate_grad(double* global_scale) {
  mle::materialize(this);
  const size_t ws_bytes = mle_sqnorm_ws_bytes(total);
  static void* ws = nullptr;
  static size_t ws_cap = 0;
  if (ws_cap < ws_bytes) {
    ws = mle::alloc_scratch(ws_bytes);
    ws_cap = ws_bytes;
  }
  check(mle_grad_sqnorm(mle::stream(), grad, total, global_scale, nullptr, ws, ws_cap), "SumSquared of " + op_name);
}

void AdamParameter::gradnorm(const double* global_scale) {
  mle::materialize(this);
  check(mle_scale_by_device(mle::stream(), grad, global_scale, 1, total), "ScalePtr of " + op_name);
}

void AdamParameter::operator=(const AdamParameter& other) {
  for (int i = 0; i < 4; ++i)
    if (dim[i] != other.dim[i]) {
      std::cout << "Shape Mismatch in equator operator of AdamParameter " << op_name << " and " << other.op_name;
      std::exit(1);
    }
  check(mle_scale_write(mle::stream(), other.output, output, 1.0f, other.total), op_name + " = " + other.op_name);
}

// ---------------------------------------------------------------------------
// small host helpers
void Dimension(graph X) {
  std::cout << "Dimensions for node: " << X->op_name << " ";
  printf("(%i x %i x %i x %i) \n", X->dim[0], X->dim[1], X->dim[2], X->dim[3]);
}
void Dimension(AdamParameter X) {
  std::cout << "Dimensions for node: " << X.op_name << " ";
  printf("(%i x %i x %i x %i) \n", X.dim[0], X.dim[1], X.dim[2], X.dim[3]);
}
void Zerograd(const AdamParameter& X) {
  auto* p = const_cast<AdamParameter*>(&X);
  mle::clip_drop(p);
  mle::zero(p->grad, p->total);
  p->grad_pending_zero = false;
}
void Zerograd(graph X) {
  mle::clip_drop(X.get());
  X->grad_src = nullptr;
  mle::zero(X->grad, X->total);
  X->grad_pending_zero = false;
}

static void print_head(NodeBackProp* X, int type, int rows_max, int cols_max) {
  if (type) mle::materialize(X);
  else mle::materialize_output(X);
  const int ch = X->dim[1], rows = X->dim[2], cols = X->dim[3];
  const long long n = std::min<long long>(X->total, (long long)ch * rows * cols);
  std::vector<float> cpu(n);
  check(mle_memcpy_d2h(cpu.data(), type ? X->grad : X->output, n * sizeof(float), mle::stream()), "print");
  std::cout << "Printing dimensions for node " << X->op_name << (type ? "->grad \n" : "->output \n");
  for (int c = 0; c < std::min(3, ch); ++c) {
    std::cout << "Channel " << c << ":\n";
    for (int r = 0; r < std::min(rows_max, rows); ++r) {
      for (int k = 0; k < std::min(cols_max, cols); ++k) std::cout << cpu[(long long)c * rows * cols + r * cols + k] << "\t";
      std::cout << "\n";
    }
    std::cout << "------------------------------\n";
  }
}
void printGPU(const graph X, const int type) { print_head(X.get(), type, X->dim[2], X->dim[3]); }
void printGPU(const AdamParameter& X, const int type) {
  print_head(const_cast<AdamParameter*>(&X), type, X.dim[2], X.dim[3]);
}
void printHeadGPU(const graph X, const int type) { print_head(X.get(), type, 5, 5); }
void printHeadGPU(const AdamParameter& X, const int type) { print_head(const_cast<AdamParameter*>(&X), type, 5, 5); }

// isNan (Engine/engine.cu:328-348): the reference's ISNAN kernel traps on a NaN
// element (Includes/kernels.h:382-392) and CheckError prints and exits.  Here
// the sum of squares of the tensor is NaN exactly when an element is NaN (an
// infinite element gives +inf, never NaN, as the reference's x != x test
// ignores infinities too); it is read back and the same message is printed.
static void nan_check(NodeBackProp* X, int type) {
  static double* acc = nullptr;
  static void* ws = nullptr;
  static size_t wcap = 0;
  if (!acc) acc = static_cast<double*>(mle::alloc_scratch(256));
  const float* p = type ? X->grad : X->output;
  if (!p || X->total <= 0) return;
  if (type) mle::materialize(X);
  else mle::materialize_output(X);
  const size_t need = mle_sqnorm_ws_bytes(X->total);
  if (wcap < need) {
    ws = mle::alloc_scratch(need);
    wcap = need;
  }
  check(mle_fill(mle::stream(), reinterpret_cast<float*>(acc), 0.0f, 2), "isNan");
  check(mle_grad_sqnorm(mle::stream(), p, X->total, acc, nullptr, ws, wcap), "isNan");
  double sum = 0.0;
  check(mle_memcpy_d2h(&sum, acc, sizeof(double), mle::stream()), "isNan");
  if (sum != sum) {
    std::cerr << "Runtime error in " << X->op_name << (type == 0 ? "output" : "grad") << " has nan value" << std::endl;
    std::exit(1);
  }
}
void isNan(graph X, const int type) { nan_check(X.get(), type); }
void isNan(const AdamParameter& X, const int type) { nan_check(const_cast<AdamParameter*>(&X), type); }

int ArgMaxToCPU(const graph& input) {
  static int32_t* d = nullptr;
  if (!d) d = static_cast<int32_t*>(mle::alloc_scratch(256));
  check(mle_argmax(mle::stream(), input->output, 1, (int)input->total, d), "ArgMax");
  int32_t out = 0;
  check(mle_memcpy_d2h(&out, d, sizeof(int32_t), mle::stream()), "ArgMax readback");
  return out;
}

// topological_sort (Engine/engine.cu:652-673): DFS post-order from the root.
graph_tree topological_sort(const graph& root) {
  std::unordered_set<NodeBackProp*> visited;
  graph_tree result;
  std::function<void(const graph&)> dfs = [&](const graph& node) {
    if (!node || visited.count(node.get())) return;
    visited.insert(node.get());
    for (const auto& in : node->inputs) dfs(in);
    result.push_back(node);
  };
  dfs(root);
  return result;
}

// ---------------------------------------------------------------------------
// GraphOperations dispatch (Engine/engine.cu:3362-3503)
double GraphOperations::GB = 0.0;
bool GraphOperations::calculate_loss = false;
float GraphOperations::loss = 0.0f;

namespace {
// Parameters reached from `nodes`, in hook order.
std::vector<AdamParameter*> collect_params(const graph_tree& nodes, bool& duplicates) {
  std::vector<AdamParameter*> ps;
  std::unordered_set<AdamParameter*> seen;
  duplicates = false;
  for (auto& n : nodes)
    for (auto* p : n->params) {
      if (!seen.insert(p).second) duplicates = true;
      ps.push_back(p);
    }
  return ps;
}

struct Span {
  float *p, *g, *m, *v;
  size_t n;
};

// Maximal runs of parameters that are contiguous in one slab.
std::vector<Span> contiguous_spans(std::vector<AdamParameter*> ps) {
  std::sort(ps.begin(), ps.end(), [](AdamParameter* a, AdamParameter* b) {
    return a->slot.slab != b->slot.slab ? a->slot.slab < b->slot.slab : a->slot.offset < b->slot.offset;
  });
  std::vector<Span> out;
  for (size_t i = 0; i < ps.size();) {
    AdamParameter* a = ps[i];
    size_t end = a->slot.offset + (((size_t)a->total + 63) & ~size_t(63));
    size_t j = i + 1;
    while (j < ps.size() && ps[j]->slot.slab == a->slot.slab && ps[j]->slot.offset == end) {
      end = ps[j]->slot.offset + (((size_t)ps[j]->total + 63) & ~size_t(63));
      ++j;
    }
    // The padding between parameters belongs to no tensor: grads there stay 0.
    const size_t n = end - a->slot.offset;
    out.push_back({a->output, a->grad, a->m, a->v, n});
    i = j;
  }
  return out;
}

void* span_ws(size_t bytes) {
  static void* ws = nullptr;
  static size_t cap = 0;
  if (cap < bytes) {
    ws = mle::alloc_scratch(bytes);
    cap = bytes;
  }
  return ws;
}
}  // namespace

void GraphOperations::clipNorm(double* global_scale) {
  bool all_hooks_known = true;
  for (auto& n : nodes)
    if (n->clipnorm && n->params.empty()) all_hooks_known = false;
  bool dup = false;
  auto ps = collect_params(nodes, dup);
  if (all_hooks_known && !ps.empty()) {
    // Deferred: the gradients read as g / s from here on (mle::clip_mark).
    mle::clip_mark(ps, global_scale);
  } else {
    mle::clip_apply_all();
    for (auto& node : nodes)
      if (node->clipnorm) node->clipnorm(global_scale);
  }
}

void GraphOperations::accumulate(double* global_scale) {
  mle::clip_apply_all();
  bool dup = false;
  auto ps = collect_params(nodes, dup);
  mle::materialize_params(ps);
  bool all_hooks_known = true;
  for (auto& n : nodes)
    if (n->accumulate && n->params.empty()) all_hooks_known = false;
  if (!all_hooks_known || dup) {
    for (auto& node : nodes)
      if (node->accumulate) node->accumulate(global_scale);
    check(mle_sqrt_scale(mle::stream(), global_scale, 1.0), "Sqrt_Scale");
    return;
  }
  // One sum per contiguous span of the arena; the last one's finishing
  // launch also applies Sqrt_Scale.
  const auto spans = contiguous_spans(ps);
  if (spans.empty()) check(mle_sqrt_scale(mle::stream(), global_scale, 1.0), "Sqrt_Scale");
  for (size_t i = 0; i < spans.size(); ++i) {
    const auto& sp = spans[i];
    const size_t ws = mle_sqnorm_ws_bytes(sp.n);
    check(mle_grad_sqnorm_ex(mle::stream(), sp.g, sp.n, global_scale, nullptr, i + 1 == spans.size() ? 1 : 0, 1.0,
                             span_ws(ws), ws),
          "SumSquared + Sqrt_Scale");
  }
}

void GraphOperations::ParameterUpdate(const graph& X, const bool show, const float lr, const bool adamw) {
  if (X) nodes = topological_sort(X);
  if (nodes.empty()) {
    printf("Warning... Nodes list is empty and parameter update cannot run.. \n");
    return;
  }
  bool dup = false;
  auto ps = collect_params(nodes, dup);
  mle::materialize_params(ps);  // a parameter no backward wrote still has its clear mark
  bool fusable = !dup && !ps.empty();
  for (auto& n : nodes)
    if (n->updateParams && n->params.empty()) fusable = false;
  for (auto* p : ps)
    if (p->t != ps[0]->t || p->b1 != ps[0]->b1 || p->b2 != ps[0]->b2 || p->epsilon != ps[0]->epsilon ||
        p->weight_decay != ps[0]->weight_decay)
      fusable = false;
  if (fusable) {
    AdamParameter* p0 = ps[0];
    // With a pending clip every gradient reads as g / s: the update divides in
    // registers and the gradients stay marked (they still read as g / s).
    const double* clip = mle::clip_view(ps);
    for (auto& sp : contiguous_spans(ps))
      check(mle_adam_update(mle::stream(), sp.p, sp.g, sp.m, sp.v, sp.n, p0->t, lr, p0->b1, p0->b2, p0->epsilon,
                            p0->weight_decay, adamw ? 1 : 0, clip),
            "AdamUpdate (fused over the parameter arena)");
    for (auto* p : ps) p->t++;
  } else {
    mle::clip_apply_all();
    for (auto& node : nodes)
      if (node->updateParams) node->updateParams(lr, adamw);
  }
  if (show)
    for (auto& node : nodes)
      if (node->updateParams) printHeadGPU(node, 1);
}

void GraphOperations::forward(const graph& X, const bool calc_loss, const bool show, const bool time,
                              const bool check_nan) {
  if (X) nodes = topological_sort(X);
  if (calc_loss) calculate_loss = true;
  if (nodes.empty()) {
    printf("Warning... Nodes list is empty and forward cannot run.. \n");
    return;
  }
  for (auto& n : nodes) n->fwd_consumers = n->fwd_key_readers = 0;
  for (auto& n : nodes)
    for (auto& in : n->inputs)
      if (in) {
        in->fwd_consumers++;
        if (n->key_target == in.get()) in->fwd_key_readers++;
      }
  for (auto& node : nodes) {
    std::chrono::high_resolution_clock::time_point t0;
    if (time) {
      mle::sync("Before " + node->op_name + " forward");
      t0 = std::chrono::high_resolution_clock::now();
    }
    if (node->forward) {
      node->forward();
      node->forward_called = true;
      if (check_nan) nan_check(node.get(), 0);
      if (show) {
        Dimension(node);
        printHeadGPU(node);
      }
    }
    if (time) {
      mle::sync("After " + node->op_name + " forward");
      const double ms =
          std::chrono::duration<double, std::milli>(std::chrono::high_resolution_clock::now() - t0).count();
      std::cout << "Time elapsed for " << node->op_name << " forward: " << ms << "ms \n";
    }
  }
  calculate_loss = false;
}

void GraphOperations::backward(const graph& X, const bool show, const bool time, const bool check_nan) {
  if (X) nodes = topological_sort(X);
  if (nodes.empty()) {
    printf("Warning... Nodes list is empty and bacward cannot run.. \n");
    return;
  }
  mle::clip_apply_all();  // parameter gradients are added into: give them their clipped values
  // An alias left by a pass without zero_grad since: its source is added into
  // below, so the node keeps its own copy.
  for (auto& n : nodes) mle::resolve_alias(n.get());
  for (auto& n : nodes) n->consumers = n->consumers_done = 0;
  for (auto& n : nodes)
    for (auto& in : n->inputs)
      if (in) in->consumers++;
  for (auto it = nodes.rbegin(); it != nodes.rend(); ++it) {
    std::chrono::high_resolution_clock::time_point t0;
    if (time) {
      mle::sync("Previous");
      t0 = std::chrono::high_resolution_clock::now();
    }
    if ((*it)->backward) {
      // The node reads its own gradient (through an alias, when it can); a
      // backward that does not know about lazy clearing may add into its
      // inputs' gradients.
      if (!(*it)->reads_grad_alias || !(*it)->grad_src) mle::materialize(it->get());
      if (!(*it)->lazy_grad_writer)
        for (auto& in : (*it)->inputs) mle::materialize(in.get());
      (*it)->backward();
      if (check_nan) nan_check(it->get(), 1);
      if (show) printHeadGPU(*it, 1);
    }
    for (auto& in : (*it)->inputs)
      if (in) in->consumers_done++;
    if (time) {
      mle::sync("After " + (*it)->op_name + " backward");
      const double ms =
          std::chrono::duration<double, std::milli>(std::chrono::high_resolution_clock::now() - t0).count();
      std::cout << "Time elapsed for " << (*it)->op_name << " backward: " << ms << "ms \n";
    }
  }
}

void GraphOperations::zero_grad(const graph& X, const bool show) {
  if (X) nodes = topological_sort(X);
  if (nodes.empty()) {
    printf("Warning... Nodes list is empty and Zero grad cannot run.. \n");
    return;
  }
  mle::clip_clear();  // the clipped gradients are being cleared anyway
  mle::ZeroBatch batch;
  for (auto it = nodes.rbegin(); it != nodes.rend(); ++it) {
    if ((*it)->zero_grad) {
      if (show) std::cout << "Zeroing gradient of" + (*it)->op_name + "\n";
      (*it)->zero_grad();
    }
  }
}

void GraphOperations::printNodes(const graph& X, const int show) {
  if (X) nodes = topological_sort(X);
  for (auto& node : nodes)
    if (node->zero_grad) {
      std::cout << "Calling Node: " << node->op_name << "\n";
      Dimension(node);
      if (show == 1) printHeadGPU(node);
      if (show == 2) printHeadGPU(node, 1);
    }
}

void GraphOperations::printParams(const graph& X, const bool show) {
  if (X) nodes = topological_sort(X);
  for (auto& node : nodes)
    if (node->printparams) node->printparams(show);
}

void GraphOperations::clear_graph(const graph& X, const bool show) {
  if (X) nodes = topological_sort(X);
  mle::sync("clear_graph");
  for (auto& node : nodes)
    if (node->free) {
      if (show) std::cout << "Freeing Node: " << node->op_name << "\n";
      node->free();
    }
  nodes.clear();
}

void GraphOperations::clean_clear_graph(const graph& X, const bool show) {
  if (X) nodes = topological_sort(X);
  mle::sync("clean_clear_graph");
  for (auto& node : nodes) {
    if (node->free) {
      if (show) std::cout << "Freeing Node: " << node->op_name << "\n";
      node->free();
    }
    if (node->serious_free) {
      if (show) std::cout << "Deleting Parameters for Node: " << node->op_name << "\n";
      node->serious_free();
    }
  }
}

// ---------------------------------------------------------------------------
// Linear (Engine/engine.cu:3505-3606).  W1 [1,1,in,out], B1 [1,1,1,out].  The
// batch and channel dimensions are folded into the GEMM's rows (the weight is
// broadcast, flags 3/0/3), so dW = X^T dY is one K = B*C*m contraction with
// the bias gradient fused into it.
Linear::Linear(const int input, const int output, const str name, const bool bias)
    : in(input), out(output), bias(bias), W1(name + " W1", 1, 1, input, output), B1(name + " B1", 1, 1, 1, output) {
  if (name != "") op_name = name;
}
void Linear::save(std::ofstream& f) const {
  W1.save(f);
  if (bias) B1.save(f);
}
void Linear::load(std::ifstream& f) {
  W1.load(f);
  if (bias) B1.load(f);
}
void Linear::operator=(const Linear& other) {
  W1 = other.W1;
  if (bias) B1 = other.B1;
}

graph Linear::forward(const graph& X) {
  if (X->dim[3] != W1.dim[2]) {
    std::cout << "Shape Mismatch in Linear Layer of " << X->op_name << ": \n";
    std::cout << "Dimensions are input " << X->op_name << "and " << op_name << ":  (" << X->dim[2] << "," << X->dim[3]
              << ") and (" << W1.dim[2] << "," << W1.dim[3] << ") \n";
    std::exit(1);
  }
  const int batch = X->dim[0], channels = X->dim[1], m = X->dim[2], n = X->dim[3], p = out;
  auto node = std::make_shared<NodeBackProp>(op_name, batch, channels, m, p, 1);
  node->lazy_grad_writer = true;
  node->reads_grad_alias = true;
  node->inputs = {X};
  GraphOperations::GB += (double)node->total * sizeof(float) / (1ULL << 30);
  const long long rows = (long long)batch * channels * m;
  AdamParameter* W = &W1;
  AdamParameter* Bb = &B1;
  const bool has_bias = bias;
  NodeBackProp* nd = node.get();
  NodeBackProp* x = X.get();
  const str name = op_name;
  node->params = has_bias ? std::vector<AdamParameter*>{W, Bb} : std::vector<AdamParameter*>{W};
  const size_t ws_f = mle_gemm_ws_bytes((int)rows, p, n, 1);
  const size_t ws_b = mle_linear_bwd_ws_bytes((int)rows, n, p, 1);
  const size_t ws_bytes = std::max(ws_f, ws_b);
  void* ws = mle::gemm_workspace(ws_bytes);
  node->forward = [=]() {
    // Y = X W + b: BCumAdd is fused into the GEMM epilogue.
    check(mle_gemm_ex(mle::stream(), 0, 0, (int)rows, p, n, 1.0f, x->output, n, 0, W->output, p, 0, 0.0f, nd->output,
                      p, 0, 1, nullptr, has_bias ? Bb->output : nullptr, ws, ws_bytes),
          "MatMul... X*W1 + B1 in " + name + " forward");
  };
  // A small product (a classifier's hidden layer) runs split along K; the
  // activation after it is then written by the reduce that completes Y
  // (mle_gemm_act_fwd), one launch less.  Large products keep the separate
  // activation pass (measured no slower than an activation epilogue).
  if ((double)rows * p <= 65536.0)
    node->forward_act = [=](int kind, float* act_out) {
      check(mle_gemm_act_fwd(mle::stream(), 0, 0, (int)rows, p, n, 1.0f, x->output, n, W->output, p, 0.0f,
                             nd->output, has_bias ? Bb->output : nullptr, kind, act_out, ws, ws_bytes),
            "MatMul... X*W1 + B1 in " + name + " forward (with the activation after it)");
    };
  if ((double)rows * p <= 4096.0)
    node->forward_xent_small = [=](const int32_t* keys, int clen, int max_clen, float* stats, int batch, float* loss,
                                   float* dlogits, float* loss_host) {
      check(mle_linear_xent_keys_small_read(mle::stream(), (int)rows, n, p, x->output, W->output,
                                            has_bias ? Bb->output : nullptr, nd->output, keys, clen, max_clen, stats,
                                            batch, loss, dlogits, loss_host),
            "MatMul... X*W1 + B1 in " + name + " forward (with the cross-entropy after it)");
    };
  node->forward_rowstats = [=](float* rowpart, int64_t ldp) {
    check(mle_gemm_rowstats(mle::stream(), 0, 0, (int)rows, p, n, 1.0f, x->output, n, W->output, p, 0.0f,
                            nd->output, p, has_bias ? Bb->output : nullptr, rowpart, ldp, ws, ws_bytes),
          "MatMul... X*W1 + B1 (with row statistics) in " + name + " forward");
  };
  node->backward = [=]() {
    // When X is an activation's output and this layer its only consumer, the
    // activation's backward (its input's gradient from dX) comes with ours.
    NodeBackProp* ai = nullptr;
    if (mle::fusion_enabled() && x->act_bwd_kind >= 0 && x->consumers == 1 && x->inputs.size() == 1 &&
        x->act_bwd_plain && x->act_bwd_plain())
      ai = x->inputs[0].get();
    if (ai) {
      const int acc_x = mle::accumulate_flag(x);
      const int acc_a = mle::accumulate_flag(ai);
      check(mle_linear_bwd_act(mle::stream(), (int)rows, n, p, x->output, mle::grad_of(nd), W->output, x->grad, acc_x,
                               W->grad, has_bias ? Bb->grad : nullptr,
                               mle::params_write_flag({W, has_bias ? Bb : nullptr}), x->act_bwd_kind, ai->output,
                               ai->grad, acc_a, ws, ws_bytes),
            "MatMul... dZ*W^T and X^T*dZ in " + name + " backward (with the activation before it)");
      x->act_bwd_done = true;
      return;
    }
    // dX (+)= dZ W^T, dW += X^T dZ, db += colsum dZ (one launch when they fit).
    check(mle_linear_bwd_ex(mle::stream(), (int)rows, n, p, 1, x->output, mle::grad_of(nd), 0, W->output, 0, x->grad,
                            mle::accumulate_flag(x), W->grad, has_bias ? Bb->grad : nullptr, 0,
                            mle::params_write_flag({W, has_bias ? Bb : nullptr}), ws, ws_bytes),
          "MatMul... dZ*W^T and X^T*dZ in " + name + " backward");
  };
  node->free = [=]() { nd->clear(); };
  node->serious_free = [=]() {};
  node->zero_grad = [=]() {
    mle::defer_zero(nd);
    mle::defer_zero(W);
    if (has_bias) mle::defer_zero(Bb);
  };
  node->accumulate = [=](double* s) {
    W->accumulate_grad(s);
    if (has_bias) Bb->accumulate_grad(s);
  };
  node->clipnorm = [=](const double* s) {
    W->gradnorm(s);
    if (has_bias) Bb->gradnorm(s);
  };
  node->updateParams = [=](const float lr, const bool adamw) {
    W->update(lr, adamw);
    if (has_bias) Bb->update(lr, adamw);
  };
  node->printparams = [=](const bool) {};
  return node;
}

// ---------------------------------------------------------------------------
// Sibling Linear fusion (see engine.h).
namespace mle {

namespace {
bool g_sibling_fusion = true;
}

void set_sibling_fusion(bool on) { g_sibling_fusion = on; }
bool fusion_enabled() { return g_sibling_fusion; }

bool fuse_sibling_linears(const std::vector<graph>& outs, const std::vector<Linear*>& layers) {
  const size_t n = outs.size();
  if (!g_sibling_fusion || n < 2 || layers.size() != n) return false;
  NodeBackProp* x = outs[0]->inputs.size() == 1 ? outs[0]->inputs[0].get() : nullptr;
  if (!x) return false;
  const Linear* l0 = layers[0];
  for (size_t i = 0; i < n; ++i) {
    if (outs[i]->inputs.size() != 1 || outs[i]->inputs[0].get() != x) return false;
    if (layers[i]->in_features() != l0->in_features() || layers[i]->out_features() != l0->out_features() ||
        layers[i]->has_bias() != l0->has_bias())
      return false;
    for (int d = 0; d < 4; ++d)
      if (outs[i]->dim[d] != outs[0]->dim[d]) return false;
  }
  // The batched launches need the outputs (and their gradients) at one
  // stride.  Node buffers come from per-size free lists, so after other
  // graphs have been freed they need not be; then the outputs and gradients
  // move into one block each (nothing has read these buffers yet: the nodes
  // were just made, and every consumer reads node->output / node->grad when
  // it runs).
  auto uniform = [&](float* NodeBackProp::*f) {
    const long long st = outs[1].get()->*f - outs[0].get()->*f;
    for (size_t i = 2; i < n; ++i)
      if (outs[i].get()->*f - outs[i - 1].get()->*f != st) return false;
    return st > 0;
  };
  for (float* NodeBackProp::*f : {&NodeBackProp::output, &NodeBackProp::grad}) {
    if (uniform(f)) continue;
    const bool grad = f == &NodeBackProp::grad;
    const size_t tot = (size_t)outs[0]->total, pad = (tot + 63) & ~size_t(63);  // the arena's 256-byte granule
    float* blk = grad ? alloc_grad(pad * n) : alloc_output(pad * n);
    for (size_t i = 0; i < n; ++i) {
      float*& ptr = outs[i].get()->*f;
      release(ptr, tot, grad);
      ptr = blk + i * pad;
      if (grad) check(mle_fill(stream(), ptr, 0.0f, tot), "Fill Kernel for Gradient");  // as a new node's
    }
  }
  // Equal strides between consecutive layers, in elements.
  auto stride_of = [&](auto get, long long& st) {
    st = (long long)(get(1) - get(0));
    if (st <= 0) return false;
    for (size_t i = 2; i < n; ++i)
      if ((long long)(get(i) - get(i - 1)) != st) return false;
    return st % 4 == 0;
  };
  long long dw, dgrad, dout, dbias = 0;
  const bool has_bias = l0->has_bias();
  if (!stride_of([&](size_t i) { return layers[i]->W1.output; }, dw) ||
      !stride_of([&](size_t i) { return outs[i]->grad; }, dgrad) ||
      !stride_of([&](size_t i) { return outs[i]->output; }, dout) ||
      (has_bias && !stride_of([&](size_t i) { return layers[i]->B1.output; }, dbias)))
    return false;
  // A parameter's gradient sits at the same offset from its value in every
  // arena region, so gradient strides equal value strides.
  for (size_t i = 1; i < n; ++i)
    if (layers[i]->W1.grad - layers[0]->W1.grad != (long long)i * dw ||
        (has_bias && layers[i]->B1.grad - layers[0]->B1.grad != (long long)i * dbias))
      return false;

  const int nl = (int)n;
  const int p = l0->out_features(), k = l0->in_features();
  const long long rows = outs[0]->total / p;
  AdamParameter* W0 = &layers[0]->W1;
  AdamParameter* B0 = &layers[0]->B1;
  NodeBackProp* o0 = outs[0].get();
  const size_t ws_f = mle_gemm_ws_bytes((int)rows, p, k, nl);
  const size_t ws_b = mle_linear_bwd_ws_bytes((int)rows, k, p, nl);
  const size_t ws_bytes = std::max(ws_f, ws_b);
  void* ws = gemm_workspace(ws_bytes);
  auto fwd_count = std::make_shared<int>(0);
  auto bwd_count = std::make_shared<int>(0);
  const str name = outs[0]->op_name;
  for (size_t i = 0; i < n; ++i) {
    // The batched backward reads the gradients at one stride: never aliased.
    outs[i]->reads_grad_alias = false;
    // Forward: the first sibling of a pass computes Y_i = X W_i + b_i for all
    // (X broadcast, weights, biases and outputs strided).
    outs[i]->forward_rowstats = nullptr;
    outs[i]->forward = [=]() {
      if ((*fwd_count)++ == 0)
        check(mle_gemm_batched_ex(stream(), 0, 0, (int)rows, p, k, 1.0f, x->output, k, 0, W0->output, p, dw, 0.0f,
                                  o0->output, p, dout, nl, nullptr, 0, has_bias ? B0->output : nullptr, dbias, ws,
                                  ws_bytes),
              "Batched X*W_i + B_i in " + name + " forward");
      if (*fwd_count == nl) *fwd_count = 0;
    };
    outs[i]->backward = [=]() {
      if (++(*bwd_count) < nl) return;
      *bwd_count = 0;
      // Every sibling's gradient is complete now (this is the last of their
      // backward calls): dX = sum_i dZ_i W_i^T, dW_i += X^T dZ_i and
      // db_i += colsum dZ_i for all siblings at once.
      std::vector<NodeBackProp*> ps;
      for (auto* l : layers) {
        ps.push_back(&l->W1);
        if (has_bias) ps.push_back(&l->B1);
      }
      check(mle_linear_bwd_ex(stream(), (int)rows, k, p, nl, x->output, o0->grad, dgrad, W0->output, dw, x->grad,
                              accumulate_flag(x), W0->grad, has_bias ? B0->grad : nullptr, dbias,
                              params_write_flag(ps), ws, ws_bytes),
            "Sibling Linear backward in " + name);
    };
  }
  return true;
}

}  // namespace mle

// ---------------------------------------------------------------------------
// Convolute2D (Engine/engine.cu:3723-3817).  W1 [out, inp, c, d], B1 [1, out, 1, 1].
Convolute2D::Convolute2D(int Input, int Output, int C, int D, int stride_, int padding, str param)
    : inp(Input),
      out(Output),
      c(C),
      d(D),
      pad(padding),
      stride(stride_),
      name(param),
      W1(param + " Weight ", Output, Input, C, D),
      B1(param + " Bias ", 1, Output, 1, 1) {}
void Convolute2D::save(std::ofstream& f) const {
  W1.save(f);
  B1.save(f);
}
void Convolute2D::load(std::ifstream& f) {
  W1.load(f);
  B1.load(f);
}

graph Convolute2D::forward(const graph& X) {
  if (X->dim[1] != inp) {
    std::cout << "Dimension Mismatch! in " << name << ": \n";
    Dimension(X);
    std::exit(1);
  }
  const int batch = X->dim[0], a = X->dim[2], b = X->dim[3];
  const int outR = (2 * pad + a - c) / stride + 1, outC = (2 * pad + b - d) / stride + 1;
  auto node = std::make_shared<NodeBackProp>(name, batch, out, outR, outC, 1);
  node->lazy_grad_writer = true;
  node->reads_grad_alias = true;
  node->inputs = {X};
  GraphOperations::GB += (double)node->total * sizeof(float) / (1ULL << 30);
  const size_t ws_bytes = mle_conv2d_wgrad_ws_bytes(batch, inp, a, b, out, c, d, pad, stride);
  void* ws = mle::alloc_scratch(ws_bytes);
  AdamParameter* W = &W1;
  AdamParameter* Bb = &B1;
  NodeBackProp* nd = node.get();
  NodeBackProp* x = X.get();
  const int inp_ = inp, out_ = out, c_ = c, d_ = d, pad_ = pad, st = stride;
  const str nm = name;
  node->params = {W, Bb};
  node->forward = [=]() {
    check(mle_conv2d_fwd(mle::stream(), x->output, W->output, Bb->output, nd->output, batch, inp_, a, b, out_, c_, d_,
                         pad_, st),
          "Forward Convolution in " + nm);
  };
  node->backward_params = [=]() {
    // dW (assigned) and db += channel sums of dZ in one launch.
    W->grad_pending_zero = false;  // the weight gradient is assigned whole (GV2D)
    check(mle_conv2d_wgrad_bias(mle::stream(), x->output, mle::grad_of(nd), W->grad, Bb->grad,
                                mle::params_write_flag({Bb}), batch, inp_, a, b, out_, c_, d_, pad_, st, ws, ws_bytes),
          "Weight and Bias Gradient in " + nm);
  };
  node->backward = [=]() {
    nd->backward_params();
    check(mle_conv2d_dgrad(mle::stream(), mle::grad_of(nd), W->output, x->grad, batch, inp_, a, b, out_, c_, d_, pad_,
                           st, mle::accumulate_flag(x)),
          "Input Gradient in " + nm);
  };
  node->zero_grad = [=]() {
    mle::defer_zero(nd);
    mle::defer_zero(W);
    mle::defer_zero(Bb);
  };
  node->free = [=]() { nd->clear(); };
  node->serious_free = [=]() {};
  node->accumulate = [=](double* s) {
    W->accumulate_grad(s);
    Bb->accumulate_grad(s);
  };
  node->clipnorm = [=](const double* s) {
    W->gradnorm(s);
    Bb->gradnorm(s);
  };
  node->updateParams = [=](const float lr, const bool adamw) {
    W->update(lr, adamw);
    Bb->update(lr, adamw);
  };
  node->printparams = [=](const bool) {};
  return node;
}

namespace mle {

bool fuse_conv_pair(const graph& y3, const Convolute2D& c3, const graph& y1, const Convolute2D& c1) {
  if (!fusion_enabled() || !y3 || !y1 || y3 == y1) return false;
  if (y3->inputs.size() != 1 || y1->inputs.size() != 1 || y3->inputs[0] != y1->inputs[0]) return false;
  if (c3.c != 3 || c3.d != 3 || c3.pad != 1 || c3.stride != 1) return false;
  if (c1.c != 1 || c1.d != 1 || c1.pad != 0 || c1.stride != 1) return false;
  if (!y3->backward_params || !y1->backward_params) return false;
  NodeBackProp* x = y3->inputs[0].get();
  const int n = x->dim[0], cin = x->dim[1], h = x->dim[2], w = x->dim[3];
  const int cout3 = c3.out, cout1 = c1.out;
  if (c3.inp != cin || c1.inp != cin) return false;
  if (!mle_conv2d_pair_supported(n, cin, h, w, cout3, cout1)) return false;
  NodeBackProp *o3 = y3.get(), *o1 = y1.get();
  const AdamParameter *W3 = &c3.W1, *B3 = &c3.B1, *W1 = &c1.W1, *B1 = &c1.B1;
  const str name = c3.name + " + " + c1.name;
  auto fwd_count = std::make_shared<int>(0);
  auto bwd_count = std::make_shared<int>(0);
  auto forward = [=]() {
    if ((*fwd_count)++ == 0)
      check(mle_conv2d_pair_fwd(stream(), x->output, n, cin, h, w, W3->output, B3->output, o3->output, cout3,
                                W1->output, B1->output, o1->output, cout1),
            "Forward Convolutions in " + name);
    if (*fwd_count == 2) *fwd_count = 0;
  };
  y3->forward = forward;
  y1->forward = forward;
  auto backward = [=](NodeBackProp* self) {
    return [=]() {
      self->backward_params();
      if (++(*bwd_count) < 2) return;
      *bwd_count = 0;
      // Both output gradients are complete (each was made readable, possibly
      // as an alias, before its node's backward) and neither has another
      // writer.
      check(mle_conv2d_pair_dgrad(stream(), x->grad, accumulate_flag(x), n, cin, h, w, grad_of(o3), W3->output, cout3,
                                  grad_of(o1), W1->output, cout1),
            "Input Gradient in " + name);
    };
  };
  y3->backward = backward(o3);
  y1->backward = backward(o1);
  return true;
}

}  // namespace mle

// ---------------------------------------------------------------------------
// Convolute2DT (Engine/engine.cu:3819-3900).  W1 [out, inp, c, d], B1 [1, out, 1, 1].
Convolute2DT::Convolute2DT(int Input, int Output, int C, int D, int stride_, int padding, str param)
    : inp(Input),
      out(Output),
      c(C),
      d(D),
      pad(padding),
      stride(stride_),
      name(param),
      W1(param + " Weight ", Output, Input, C, D),
      B1(param + " Bias ", 1, Output, 1, 1) {}
void Convolute2DT::save(std::ofstream& f) const {
  W1.save(f);
  B1.save(f);
}
void Convolute2DT::load(std::ifstream& f) {
  W1.load(f);
  B1.load(f);
}

graph Convolute2DT::forward(const graph& X) {
  if (X->dim[1] != inp) {
    std::cout << "Dimension Mismatch! in " << name << ": \n";
    Dimension(X);
    std::cout << "Actual input (Batch x depth): (" << X->dim[0] << "x" << X->dim[1] << ") \n";
    std::cout << "Expected input (Batch x depth): (" << X->dim[0] << "x" << inp << ") \n";
    std::exit(1);
  }
  const int batch = X->dim[0], ih = X->dim[2], iw = X->dim[3];
  const int oh = (ih - 1) * stride - 2 * pad + c, ow = (iw - 1) * stride - 2 * pad + d;
  if (oh <= 0 || ow <= 0) {
    std::cout << "Non-positive output size in " << name << "\n";
    std::exit(1);
  }
  auto node = std::make_shared<NodeBackProp>(name, batch, out, oh, ow, 1);
  node->lazy_grad_writer = true;
  node->inputs = {X};
  GraphOperations::GB += (double)(node->total + W1.total + B1.total) * sizeof(float) / (1ULL << 30);
  // The convolution this is the adjoint of maps [batch, out, oh, ow] to
  // [batch, inp, ih, iw] with weights [inp, out, c, d] (W1 swapped).
  const size_t wn = (size_t)W1.total;
  float* wt = static_cast<float*>(mle::alloc_scratch(2 * wn * sizeof(float)));  // swapped weight | its gradient
  float* wtg = wt + wn;
  const size_t ws_bytes = mle_conv2d_wgrad_ws_bytes(batch, out, oh, ow, inp, c, d, pad, stride);
  void* ws = mle::alloc_scratch(ws_bytes);
  AdamParameter* W = &W1;
  AdamParameter* Bb = &B1;
  NodeBackProp* nd = node.get();
  NodeBackProp* x = X.get();
  const int inp_ = inp, out_ = out, c_ = c, d_ = d, pad_ = pad, st = stride;
  const str nm = name;
  node->params = {W, Bb};
  node->forward = [=]() {
    check(mle_weight_swap(mle::stream(), W->output, wt, out_, inp_, c_ * d_, 0), "Weight swap in " + nm);
    check(mle_conv2d_dgrad(mle::stream(), x->output, wt, nd->output, batch, out_, oh, ow, inp_, c_, d_, pad_, st, 0),
          "ConvTranspose2D Forward in " + nm);
    check(mle_broadcast_channel_add(mle::stream(), nd->output, Bb->output, nd->output, batch, out_, (size_t)oh * ow),
          "ConvTranspose2D bias in " + nm);
  };
  node->backward = [=]() {
    mle::materialize(W);
    mle::materialize(Bb);
    check(mle_conv2d_wgrad(mle::stream(), nd->grad, x->output, wtg, batch, out_, oh, ow, inp_, c_, d_, pad_, st, ws,
                           ws_bytes),
          "Weight Gradient in " + nm);
    check(mle_weight_swap(mle::stream(), wtg, W->grad, inp_, out_, c_ * d_, 0), "Weight gradient swap in " + nm);
    check(mle_channel_sum(mle::stream(), nd->grad, batch, out_, (size_t)oh * ow, out_, Bb->grad),
          "Bias Gradient in " + nm);
    mle::accumulate_flag(x);  // assigned, as CVT2D_GradInput does
    check(mle_conv2d_fwd(mle::stream(), nd->grad, wt, nullptr, x->grad, batch, out_, oh, ow, inp_, c_, d_, pad_, st),
          "Input Gradient in " + nm);
  };
  node->zero_grad = [=]() {
    mle::defer_zero(nd);
    mle::defer_zero(W);
    mle::defer_zero(Bb);
  };
  node->free = [=]() { nd->clear(); };
  node->serious_free = [=]() {};
  node->accumulate = [=](double* s) {
    W->accumulate_grad(s);
    Bb->accumulate_grad(s);
  };
  node->clipnorm = [=](const double* s) {
    W->gradnorm(s);
    Bb->gradnorm(s);
  };
  node->updateParams = [=](const float lr, const bool adamw) {
    W->update(lr, adamw);
    Bb->update(lr, adamw);
  };
  node->printparams = [=](const bool) {};
  return node;
}

// ---------------------------------------------------------------------------
// Embedding
Embedding::Embedding(int vocab_, int dim_, const str name) : vocab(vocab_), dim(dim_), E(name, 1, 1, vocab_, dim_) {}
void Embedding::save(std::ofstream& f) const { E.save(f); }
void Embedding::load(std::ifstream& f) { E.load(f); }

graph Embedding::forward(const int32_t* keys, int batch, int clen, int max_clen) {
  auto node = std::make_shared<NodeBackProp>(E.op_name + " lookup", batch, 1, clen, dim, 1);
  node->lazy_grad_writer = true;
  keys_ = keys;
  batch_ = batch;
  clen_ = clen;
  max_clen_ = max_clen;
  ws_bytes_ = mle_embed_scatter_ws_bytes(batch, clen);
  ws_ = mle::alloc_scratch(ws_bytes_);
  AdamParameter* T = &E;
  NodeBackProp* nd = node.get();
  const int V = vocab, D = dim;
  void* ws = ws_;
  const size_t wsb = ws_bytes_;
  // The forward's gather also indexes the tokens of each table row (this
  // node's own index: the keys do not change before its backward), so the
  // backward only sums rows.  Vocabularies above the index's limit scan the
  // keys in the backward instead.
  const size_t ixb = mle_embed_index_bytes(batch, clen, V);
  void* index = ixb ? mle::alloc_scratch(ixb) : nullptr;
  node->params = {T};
  node->forward = [=]() {
    if (index)
      check(mle_embed_gather_indexed(mle::stream(), nd->output, T->output, keys, batch, clen, max_clen, D, V, index, ixb),
            "GatherEmbeddings");
    else
      check(mle_embed_gather(mle::stream(), nd->output, T->output, keys, batch, clen, max_clen, D), "GatherEmbeddings");
  };
  node->backward = [=]() {
    if (index)
      check(mle_embed_grad_indexed(mle::stream(), T->grad, nd->grad, index, batch, clen, D, V,
                                   mle::params_write_flag({T})),
            "Embedding gradient");
    else
      check(mle_embed_grad(mle::stream(), T->grad, nd->grad, keys, batch, clen, max_clen, D, V,
                           mle::params_write_flag({T}), ws, wsb),
            "Embedding gradient");
  };
  node->zero_grad = [=]() {
    mle::defer_zero(nd);
    mle::defer_zero(T);
  };
  node->free = [=]() { nd->clear(); };
  node->accumulate = [=](double* s) { T->accumulate_grad(s); };
  node->clipnorm = [=](const double* s) { T->gradnorm(s); };
  node->updateParams = [=](const float lr, const bool adamw) { T->update(lr, adamw); };
  return node;
}

namespace {
constexpr uint32_t kTembMagic = 0x54454D42u;  // "TEMB"
constexpr uint32_t kTembVersion = 1u;

// Header and vocabulary of a TEMB file; false (after printing) on a bad file.
bool temb_read_header(std::ifstream& f, const str& who, int dim, std::vector<std::pair<str, int>>& words) {
  uint32_t magic = 0, version = 0;
  f.read(reinterpret_cast<char*>(&magic), sizeof(magic));
  f.read(reinterpret_cast<char*>(&version), sizeof(version));
  if (!f || magic != kTembMagic) {
    std::cerr << who << " -- bad magic number; not a TEMB file\n";
    return false;
  }
  if (version != kTembVersion) {
    std::cerr << who << " -- unsupported version " << version << "\n";
    return false;
  }
  int saved_dim = 0, n = 0;
  f.read(reinterpret_cast<char*>(&saved_dim), sizeof(saved_dim));
  f.read(reinterpret_cast<char*>(&n), sizeof(n));
  if (!f || n < 0) {
    std::cerr << who << " -- read error in the header\n";
    return false;
  }
  if (saved_dim != dim) {
    std::cerr << who << " -- embed_dim mismatch: file=" << saved_dim << " object=" << dim << "\n";
    return false;
  }
  words.clear();
  words.reserve(n);
  for (int i = 0; i < n; ++i) {
    uint32_t wlen = 0;
    f.read(reinterpret_cast<char*>(&wlen), sizeof(wlen));
    str w(wlen, '\0');
    if (wlen) f.read(&w[0], wlen);
    int idx = 0;
    f.read(reinterpret_cast<char*>(&idx), sizeof(idx));
    if (!f) {
      std::cerr << who << " -- read error in the vocabulary\n";
      return false;
    }
    words.emplace_back(std::move(w), idx);
  }
  return true;
}
}  // namespace

void Embedding::save(const str& filepath, const std::unordered_map<str, int>& words) const {
  std::ofstream f(filepath, std::ios::binary);
  if (!f.is_open()) {
    std::cerr << "TextualEmbedding::save -- could not open '" << filepath << "' for writing\n";
    return;
  }
  const int n = (int)words.size();
  if (n > vocab) {
    std::cerr << "TextualEmbedding::save -- " << n << " words for a table of " << vocab << " rows\n";
    return;
  }
  f.write(reinterpret_cast<const char*>(&kTembMagic), sizeof(kTembMagic));
  f.write(reinterpret_cast<const char*>(&kTembVersion), sizeof(kTembVersion));
  f.write(reinterpret_cast<const char*>(&dim), sizeof(dim));
  f.write(reinterpret_cast<const char*>(&n), sizeof(n));
  for (const auto& [word, idx] : words) {
    const uint32_t wlen = (uint32_t)word.size();
    f.write(reinterpret_cast<const char*>(&wlen), sizeof(wlen));
    f.write(word.data(), wlen);
    f.write(reinterpret_cast<const char*>(&idx), sizeof(idx));
  }
  // Rows 0 .. n-1 of the table, one device-to-host copy.
  std::vector<float> host((size_t)n * dim);
  if (n) check(mle_memcpy_d2h(host.data(), E.output, host.size() * sizeof(float), mle::stream()), "TEMB save");
  f.write(reinterpret_cast<const char*>(host.data()), (std::streamsize)(host.size() * sizeof(float)));
  if (!f.good()) std::cerr << "TextualEmbedding::save -- write error on '" << filepath << "'\n";
}

int Embedding::load(const str& filepath, std::unordered_map<str, int>& words) {
  const str who = "TextualEmbedding::load";
  std::ifstream f(filepath, std::ios::binary);
  if (!f.is_open()) {
    std::cerr << who << " -- could not open '" << filepath << "'\n";
    return -1;
  }
  std::vector<std::pair<str, int>> saved;
  if (!temb_read_header(f, who, dim, saved)) return -1;
  const int n = (int)saved.size();
  if (n > vocab) {
    std::cerr << who << " -- saved vocab (" << n << ") exceeds MAX_VOCAB_SIZE (" << vocab << ")\n";
    return -1;
  }
  std::vector<float> host((size_t)n * dim);
  f.read(reinterpret_cast<char*>(host.data()), (std::streamsize)(host.size() * sizeof(float)));
  if (!f.good()) {
    std::cerr << who << " -- read error on '" << filepath << "'\n";
    return -1;
  }
  words.clear();
  for (auto& [w, idx] : saved) words[w] = idx;
  if (n) check(mle_memcpy_h2d(E.output, host.data(), host.size() * sizeof(float), mle::stream()), "TEMB load");
  return n;
}

int Embedding::load_replace(const str& filepath, const std::unordered_map<str, int>& words) {
  const str who = "TextualEmbedding::load_replace";
  std::ifstream f(filepath, std::ios::binary);
  if (!f.is_open()) {
    std::cerr << who << " -- could not open '" << filepath << "'\n";
    return -1;
  }
  std::vector<std::pair<str, int>> saved;
  if (!temb_read_header(f, who, dim, saved)) return -1;
  // (local row, saved row) for the words both vocabularies hold, in file-row order.
  std::vector<std::pair<int, int>> match;
  for (const auto& [w, sidx] : saved) {
    auto it = words.find(w);
    if (it != words.end() && it->second >= 0 && it->second < vocab) match.emplace_back(it->second, sidx);
  }
  if (match.empty()) return 0;
  std::sort(match.begin(), match.end(), [](const auto& a, const auto& b) { return a.second < b.second; });
  std::vector<float> row(dim);
  size_t cur = 0;
  int replaced = 0;
  for (int s = 0; s < (int)saved.size() && cur < match.size(); ++s) {
    f.read(reinterpret_cast<char*>(row.data()), (std::streamsize)(dim * sizeof(float)));
    if (!f.good()) {
      std::cerr << who << " -- read error at embedding row " << s << "\n";
      return replaced;
    }
    while (cur < match.size() && match[cur].second == s) {
      check(mle_memcpy_h2d(E.output + (size_t)match[cur].first * dim, row.data(), dim * sizeof(float), mle::stream()),
            "TEMB load_replace");
      ++replaced;
      ++cur;
    }
    while (cur < match.size() && match[cur].second < s) ++cur;  // saved row index outside the file
  }
  return replaced;
}

void Embedding::UpdateSGD(const graph& X, float lr) {
  check(mle_embed_scatter_add(mle::stream(), E.output, X->grad, keys_, batch_, clen_, max_clen_, dim, vocab, -lr, ws_,
                              ws_bytes_),
        "Key Update in Embedding Space update");
}
