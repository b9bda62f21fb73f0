// libmalus_hip runtime core: the device context, tensor handles and
// refcounts, the size-bucketed device pool, stream-ordered execution with
// pending-read flushes, host I/O, RNG builtins, staging buffers and the
// bench timer.  Drop-in for crates/malus-runtime/src/metal.rs (context,
// pool, alloc/free, barrier, reshape, RNG), buffer.rs, bench.rs and lib.rs.
//
// Execution model (replaces ADR-0035's shared command buffer): every op is
// enqueued on ONE in-order HIP stream.  Stream order makes a freed buffer
// immediately reusable by later work, so the pool needs no generation
// gating; a host read waits only when the tensor's last write has not
// completed (write_seq > completed_seq), like metal.rs:244-252.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

#include "common.h"
#include "api.h"

namespace malus {

// ============================================================================
// errors
// ============================================================================
static std::atomic<int> g_abort_on_error{1};
thread_local int g_api_depth = 0;
static thread_local std::string g_last_error;

size_t dtype_size(int32_t tag) {
  switch (tag) {
    case F32: case I32: case U32: return 4;
    case F16: case BF16: case I16: case U16: return 2;
    case I8: case U8: return 1;
    case I64: case U64: return 8;
  }
  fail("malus: unknown dtype tag %d", tag);
}

void fail(const char* fmt, ...) {
  char buf[2048];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  if (g_abort_on_error.load()) {
    fprintf(stderr, "%s\n", buf);
    fflush(stderr);
    std::abort();
  }
  throw MalusError(buf);
}

void set_last_error(const char* msg) { g_last_error = msg; }

void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess) fail("malus: HIP error %s (%d) in %s", hipGetErrorString(e), (int)e, what);
}

std::string shape_str(const TensorBuffer* t) {
  std::string s = "[";
  for (int i = 0; i < t->ndim; ++i) {
    if (i) s += ", ";
    s += std::to_string(t->shape[i]);
  }
  return s + "]";
}

// ============================================================================
// counters (runtime/lib.rs:1-94)
// ============================================================================
static std::atomic<int64_t> g_retain{0}, g_release{0}, g_alloc{0};
static std::atomic<uint32_t> g_gradcheck_bits{0};

// ============================================================================
// context
// ============================================================================
namespace {

struct Staging {
  char* base = nullptr;
  size_t cap = 0, head = 0;
  struct Region { size_t beg, end; hipEvent_t ev; };
  std::deque<Region> inflight;
  std::vector<hipEvent_t> spare;
};

struct Pool {
  std::mutex mu;
  std::unordered_map<size_t, std::vector<void*>> free_lists;
  int64_t hits = 0, misses = 0, pooled_bytes = 0, live_bytes = 0, peak_bytes = 0;
  std::map<size_t, uint64_t> histogram;
  // HIP graph capture: every buffer handed out while a capture is recorded
  // (capture_owner != 0) belongs to that graph afterwards.  A graph's buffer
  // that is freed goes to the graph's own list, never back to the free
  // lists, so no later allocation can share memory the graph's replays write.
  int capture_owner = 0;
  std::unordered_map<void*, std::pair<int, size_t>> reserved;       // ptr -> (graph, bucket)
  std::unordered_map<int, std::vector<std::pair<void*, size_t>>> reserved_free;  // graph -> its freed buffers
};

struct Context {
  int device = 0;
  hipStream_t stream = nullptr;
  Staging staging;
  Pool pool;
  int32_t* err_flag = nullptr;  // device int[4]
  std::atomic<uint64_t> seq{0}, completed{0};
  bool sync_dispatch = false;
  bool histogram = false;
  int64_t budget = -1;  // -1: derive from env
  int64_t fail_alloc_after = -1;  // fault injection for error-path tests: -1 off
};

Context* g_ctx = nullptr;
std::once_flag g_once;

Context& ctx() {
  ensure_init();
  return *g_ctx;
}

size_t bucket_size(size_t bytes) {
  if (bytes == 0) bytes = 1;  // metal.rs:384-387: zero-length tensors get a placeholder
  if (bytes <= 4096) return (bytes + 255) / 256 * 256;
  size_t p2 = 1;
  while (p2 < bytes) p2 <<= 1;
  size_t gran = p2 / 16;  // <= 6.25 % rounding
  return (bytes + gran - 1) / gran * gran;
}

int64_t mem_budget(Context& c) {
  if (c.budget >= 0) return c.budget;
  const char* e = getenv("MALUS_MEM_BUDGET_MB");
  if (e) {
    long long mb = atoll(e);
    if (mb == 0) return INT64_MAX;
    if (mb > 0) return (int64_t)mb << 20;
  }
  return INT64_MAX;  // 288 GB of HBM: no artificial ceiling by default
}

void trim_pool(Context& c) {
  // caller holds pool.mu; frees every pooled buffer after draining the stream
  MALUS_HIP(hipStreamSynchronize(c.stream));
  for (auto& kv : c.pool.free_lists)
    for (void* p : kv.second) {
      MALUS_HIP(hipFree(p));
      c.pool.pooled_bytes -= (int64_t)kv.first;
    }
  c.pool.free_lists.clear();
}

}  // namespace

void ensure_init() {
  std::call_once(g_once, [] {
    auto* c = new Context();
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) fail("malus: no HIP device available (hipGetDeviceCount: %s, count %d)", hipGetErrorString(e), n);
    MALUS_HIP(hipGetDevice(&c->device));
    MALUS_HIP(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
    c->staging.cap = 64u << 20;
    MALUS_HIP(hipHostMalloc(reinterpret_cast<void**>(&c->staging.base), c->staging.cap, hipHostMallocDefault));
    MALUS_HIP(hipMalloc(reinterpret_cast<void**>(&c->err_flag), 4 * sizeof(int32_t)));
    MALUS_HIP(hipMemset(c->err_flag, 0, 4 * sizeof(int32_t)));
    const char* sd = getenv("MALUS_SYNC_DISPATCH");
    c->sync_dispatch = sd && std::string(sd) == "1";
    const char* hg = getenv("MALUS_ALLOC_HISTOGRAM");
    c->histogram = hg && std::string(hg) == "1";
    g_ctx = c;
    noalloc_init_device(c->device);
    register_default_backward_fns();
  });
}

hipStream_t stream() { return ctx().stream; }
int32_t* device_error_flag() { return ctx().err_flag; }

static void check_device_errors(Context& c) {
  int32_t flags[4];
  MALUS_HIP(hipMemcpy(flags, c.err_flag, sizeof(flags), hipMemcpyDeviceToHost));
  if (flags[0] || flags[1] || flags[2] || flags[3]) {
    MALUS_HIP(hipMemset(c.err_flag, 0, 4 * sizeof(int32_t)));
    if (flags[0] == 1) fail("malus: embedding index out of range (detected on the GPU)");
    if (flags[0] == 2) fail("malus: cross_entropy target index out of range (detected on the GPU)");
    fail("malus: device-side error flag %d", flags[0]);
  }
}

void sync_all() {
  Context& c = ctx();
  uint64_t upto = c.seq.load();
  hipError_t e = hipStreamSynchronize(c.stream);
  if (e != hipSuccess)
    fail("malus: GPU stream failed: %s (set MALUS_SYNC_DISPATCH=1 to attribute the failing op)", hipGetErrorString(e));
  c.completed.store(upto);
  check_device_errors(c);
}

uint64_t enqueue_mark(const char* op_name) {
  Context& c = ctx();
  uint64_t s = ++c.seq;
  static const bool trace = getenv("MALUS_OP_TRACE") != nullptr;  // one line per enqueued op (instrumentation)
  if (trace) fprintf(stderr, "malus op %s\n", op_name);
  if (c.sync_dispatch) {
    hipError_t e = hipStreamSynchronize(c.stream);
    if (e != hipSuccess) fail("malus: GPU op '%s' failed: %s", op_name, hipGetErrorString(e));
    c.completed.store(s);
    check_device_errors(c);
  }
  return s;
}

void flush_if_pending(TensorBuffer* t) {
  if (!t) return;
  if (t->write_seq > ctx().completed.load()) sync_all();
}

// ============================================================================
// pool
// ============================================================================
void* pool_alloc(size_t bytes, size_t* bucket_out) {
  Context& c = ctx();
  size_t b = bucket_size(bytes);
  std::lock_guard<std::mutex> lk(c.pool.mu);
  if (c.fail_alloc_after >= 0 && c.fail_alloc_after-- == 0) fail("malus: injected allocation failure (%zu bytes)", b);
  if (c.histogram) c.pool.histogram[b]++;
  auto it = c.pool.free_lists.find(b);
  if (it != c.pool.free_lists.end() && !it->second.empty()) {
    void* p = it->second.back();
    it->second.pop_back();
    c.pool.hits++;
    c.pool.pooled_bytes -= (int64_t)b;
    c.pool.live_bytes += (int64_t)b;
    if (c.pool.capture_owner) c.pool.reserved[p] = {c.pool.capture_owner, b};
    *bucket_out = b;
    return p;
  }
  c.pool.misses++;
  if (c.pool.live_bytes + c.pool.pooled_bytes + (int64_t)b > mem_budget(c) && c.pool.pooled_bytes > 0) trim_pool(c);
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, b);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    trim_pool(c);  // release cached buffers and retry once
    e = hipMalloc(&p, b);
    if (e != hipSuccess) fail("malus: device allocation of %zu bytes failed: %s", b, hipGetErrorString(e));
  }
  c.pool.live_bytes += (int64_t)b;
  c.pool.peak_bytes = std::max(c.pool.peak_bytes, c.pool.live_bytes + c.pool.pooled_bytes);
  if (c.pool.capture_owner) c.pool.reserved[p] = {c.pool.capture_owner, b};
  *bucket_out = b;
  return p;
}

void pool_free(void* p, size_t bucket) {
  if (!p) return;
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.pool.mu);
  auto r = c.pool.reserved.find(p);
  if (r != c.pool.reserved.end() && r->second.first != c.pool.capture_owner) {
    // a graph's buffer, freed outside that graph's capture: kept for the
    // graph (it stays counted as live)
    c.pool.reserved_free[r->second.first].emplace_back(p, bucket);
    return;
  }
  c.pool.live_bytes -= (int64_t)bucket;
  c.pool.pooled_bytes += (int64_t)bucket;
  c.pool.free_lists[bucket].push_back(p);
}

void pool_capture_begin(int graph) {
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.pool.mu);
  if (c.pool.capture_owner) fail("malus: a graph capture is already being recorded");
  c.pool.capture_owner = graph;
}

void pool_capture_end(int graph) {
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.pool.mu);
  if (c.pool.capture_owner != graph) fail("malus: pool_capture_end for a graph that is not capturing");
  c.pool.capture_owner = 0;
  // buffers the capture freed sit in the free lists: move them to the graph
  for (auto& fl : c.pool.free_lists) {
    auto& v = fl.second;
    for (size_t i = 0; i < v.size();) {
      auto r = c.pool.reserved.find(v[i]);
      if (r != c.pool.reserved.end() && r->second.first == graph) {
        c.pool.reserved_free[graph].emplace_back(v[i], fl.first);
        c.pool.pooled_bytes -= (int64_t)fl.first;
        c.pool.live_bytes += (int64_t)fl.first;
        v[i] = v.back();
        v.pop_back();
      } else {
        ++i;
      }
    }
  }
}

// The graph is gone: its freed buffers return to the free lists, and its
// live ones return there when their tensors are released.
void pool_release_graph(int graph) {
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.pool.mu);
  for (auto& q : c.pool.reserved_free[graph]) {
    c.pool.free_lists[q.second].push_back(q.first);
    c.pool.live_bytes -= (int64_t)q.second;
    c.pool.pooled_bytes += (int64_t)q.second;
  }
  c.pool.reserved_free.erase(graph);
  for (auto it = c.pool.reserved.begin(); it != c.pool.reserved.end();) {
    if (it->second.first == graph) it = c.pool.reserved.erase(it);
    else ++it;
  }
}

// ============================================================================
// tensors
// ============================================================================
// The reference's dtypes (metal.rs:368-377), plus bf16 for the autocast
// paths (docs/adr/0037-bf16-autocast.md consequences: the Bf16 tag stops
// panicking on the autocast-covered paths only; tensor_alloc_gpu keeps the
// reference's check).
TensorBuffer* alloc_tensor(int32_t dtype, const size_t* shape, int ndim) {
  if (dtype != F32 && dtype != I32 && dtype != I64 && dtype != BF16)
    fail("malus: unsupported dtype tag %d; supported: f32, i32, i64", dtype);
  if (ndim < 0 || ndim > kMaxRank) fail("malus: tensor rank %d exceeds %d", ndim, kMaxRank);
  auto* t = new TensorBuffer();
  t->dtype = dtype;
  t->ndim = ndim;
  size_t n = 1;
  for (int i = 0; i < ndim; ++i) { t->shape[i] = shape[i]; n *= shape[i]; }
  t->len = n;
  auto* st = new Storage();
  st->ptr = pool_alloc(n * dtype_size(dtype), &st->bytes);
  st->aliases = 1;
  t->st = st;
  g_alloc++;
  return t;
}

TensorBuffer* alloc_like(const TensorBuffer* t) { return alloc_tensor(t->dtype, t->shape, t->ndim); }

TensorBuffer* alloc_f32(std::initializer_list<size_t> shape) {
  size_t s[kMaxRank];
  int n = 0;
  for (size_t v : shape) s[n++] = v;
  return alloc_tensor(F32, s, n);
}

TensorBuffer* alloc_virtual(int32_t dtype, const size_t* shape, int ndim) {
  if (ndim < 0 || ndim > kMaxRank) fail("malus: tensor rank %d exceeds %d", ndim, kMaxRank);
  auto* t = new TensorBuffer();
  t->dtype = dtype;
  t->ndim = ndim;
  size_t n = 1;
  for (int i = 0; i < ndim; ++i) { t->shape[i] = shape[i]; n *= shape[i]; }
  t->len = n;
  auto* st = new Storage();
  st->ptr = nullptr;
  st->bytes = 0;
  st->aliases = 1;
  t->st = st;
  g_alloc++;
  return t;
}

TensorBuffer* make_alias(TensorBuffer* src, const size_t* shape, int ndim) {
  // reshape_to, metal.rs:1385-1403: same storage, inherited pending state
  auto* t = new TensorBuffer();
  t->dtype = src->dtype;
  t->ndim = ndim;
  t->len = src->len;
  for (int i = 0; i < ndim; ++i) t->shape[i] = shape[i];
  t->st = src->st;
  t->st->aliases++;
  t->write_seq = src->write_seq;
  return t;
}

void retain(TensorBuffer* t) {
  if (!t) return;
  g_retain++;
  t->rc.fetch_add(1);
}

void release(TensorBuffer* t) {
  if (!t) return;
  g_release++;
  int64_t prev = t->rc.fetch_sub(1);
  if (prev <= 0)
    fail("malus: over-release of tensor handle %#llx (refcount already zero) - likely a borrow-inference or tape-retain bug",
         (unsigned long long)H(t));
  if (prev == 1) {
    tape_on_release(H(t));  // metal.rs:534: leaf registry cleanup first
    if (t->bf16_copy) release(t->bf16_copy);
    Storage* st = t->st;
    if (--st->aliases == 0) {
      pool_free(st->ptr, st->bytes);
      delete st;
    }
    delete t;
  }
}

// ============================================================================
// host <-> device
// ============================================================================
void upload(void* dst, const void* src, size_t bytes) {
  if (!bytes) return;
  Context& c = ctx();
  Staging& sg = c.staging;
  size_t need = (bytes + 255) / 256 * 256;
  if (need > sg.cap / 2) {  // large: copy directly and wait for it
    MALUS_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c.stream));
    MALUS_HIP(hipStreamSynchronize(c.stream));
    return;
  }
  if (sg.head + need > sg.cap) sg.head = 0;
  while (!sg.inflight.empty()) {
    auto& f = sg.inflight.front();
    bool overlap = f.beg < sg.head + need && sg.head < f.end;
    if (!overlap) break;
    MALUS_HIP(hipEventSynchronize(f.ev));
    sg.spare.push_back(f.ev);
    sg.inflight.pop_front();
  }
  char* stage = sg.base + sg.head;
  memcpy(stage, src, bytes);
  MALUS_HIP(hipMemcpyAsync(dst, stage, bytes, hipMemcpyHostToDevice, c.stream));
  hipEvent_t ev;
  if (sg.spare.empty()) MALUS_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
  else { ev = sg.spare.back(); sg.spare.pop_back(); }
  MALUS_HIP(hipEventRecord(ev, c.stream));
  sg.inflight.push_back({sg.head, sg.head + need, ev});
  sg.head += need;
}

void materialize_upper_tiles(TensorBuffer* t) {
  if (!t || !t->st || !t->st->upper_unwritten_t) return;
  const size_t tt = t->st->upper_unwritten_t;
  k::attn_zero_upper_tiles(t->f32(), t->len / (tt * tt), tt, stream());
  t->st->upper_unwritten_t = 0;
  t->write_seq = enqueue_mark("attn_zero_upper");
}

void download(void* dst, const TensorBuffer* t, size_t bytes) {
  materialize_upper_tiles(const_cast<TensorBuffer*>(t));
  flush_if_pending(const_cast<TensorBuffer*>(t));
  if (!bytes) return;
  if (!t->st->ptr) fail("malus: tensor %s has no device storage (an intermediate of a fused kernel)", shape_str(t).c_str());
  Context& c = ctx();
  MALUS_HIP(hipMemcpyAsync(dst, t->data(), bytes, hipMemcpyDeviceToHost, c.stream));
  MALUS_HIP(hipStreamSynchronize(c.stream));
}

// ============================================================================
// RNG: Philox4x32-10 (metal.rs:1690-1759)
// ============================================================================
void philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
  uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3], k0 = key[0], k1 = key[1];
  for (int r = 0; r < 10; ++r) {
    uint64_t p0 = (uint64_t)c0 * 0xD2511F53u, p1 = (uint64_t)c2 * 0xCD9E8D57u;
    uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0, n1 = (uint32_t)p1;
    uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1, n3 = (uint32_t)p0;
    c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

static thread_local uint64_t t_rng_calls = 0;  // RANDN_CALL_COUNTER (metal.rs:1713-1715)
uint64_t rng_next_call() { return t_rng_calls++; }

// Rust `{}` (Display) of an f32: shortest round-trip digits, positional form.
static std::string rust_f32(float v) {
  if (std::isnan(v)) return "NaN";
  if (std::isinf(v)) return v > 0 ? "inf" : "-inf";
  if (v == 0.0f) return std::signbit(v) ? "-0" : "0";
  char buf[64];
  int prec = 1;
  for (; prec <= 9; ++prec) {
    snprintf(buf, sizeof(buf), "%.*e", prec - 1, (double)v);
    if (strtof(buf, nullptr) == v) break;
  }
  // buf = [-]d.ddde[+-]XX
  std::string s(buf);
  bool neg = s[0] == '-';
  if (neg) s = s.substr(1);
  size_t epos = s.find('e');
  int exp10 = atoi(s.c_str() + epos + 1);
  std::string digits;
  for (size_t i = 0; i < epos; ++i) if (s[i] != '.') digits += s[i];
  while (digits.size() > 1 && digits.back() == '0') digits.pop_back();
  std::string out;
  int point = exp10 + 1;  // digits before the decimal point
  if (point <= 0) {
    out = "0." + std::string((size_t)(-point), '0') + digits;
  } else if ((size_t)point >= digits.size()) {
    out = digits + std::string((size_t)point - digits.size(), '0');
  } else {
    out = digits.substr(0, (size_t)point) + "." + digits.substr((size_t)point);
  }
  return neg ? "-" + out : out;
}

template <class V, class F>
static void print_nd(const V* data, const size_t* shape, int ndim, size_t offset, F fmt) {
  if (ndim == 0) { fputs(fmt(data[offset]).c_str(), stdout); return; }
  size_t stride = 1;
  for (int i = 1; i < ndim; ++i) stride *= shape[i];
  fputc('[', stdout);
  for (size_t i = 0; i < shape[0]; ++i) {
    if (i) fputs(", ", stdout);
    if (ndim == 1) fputs(fmt(data[offset + i]).c_str(), stdout);
    else print_nd(data, shape + 1, ndim - 1, offset + i * stride, fmt);
  }
  fputc(']', stdout);
}

// ============================================================================
// per-kernel timing
// ============================================================================
struct KTimer {
  const char* cls;
  hipEvent_t e0, e1;
  double units;
};
static std::atomic<bool> g_ktimer_on{false};
static std::vector<KTimer*> g_ktimers;
static std::vector<KTimer*> g_ktimer_spare;
static std::mutex g_ktimer_mu;

KTimer* ktimer_begin(const char* cls) {
  if (!g_ktimer_on.load()) return nullptr;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  MALUS_HIP(hipStreamIsCapturing(stream(), &cap));
  if (cap != hipStreamCaptureStatusNone) return nullptr;  // no event nodes in a captured step
  std::lock_guard<std::mutex> lk(g_ktimer_mu);
  KTimer* t;
  if (g_ktimer_spare.empty()) {
    t = new KTimer();
    MALUS_HIP(hipEventCreate(&t->e0));
    MALUS_HIP(hipEventCreate(&t->e1));
  } else {
    t = g_ktimer_spare.back();
    g_ktimer_spare.pop_back();
  }
  t->cls = cls;
  MALUS_HIP(hipEventRecord(t->e0, stream()));
  return t;
}

void ktimer_end(KTimer* t, double units) {
  if (!t) return;
  MALUS_HIP(hipEventRecord(t->e1, stream()));
  t->units = units;
  std::lock_guard<std::mutex> lk(g_ktimer_mu);
  g_ktimers.push_back(t);
}

}  // namespace malus

using namespace malus;

// ============================================================================
// C ABI
// ============================================================================
extern "C" {

int malus_set_abort_on_error(int on) { return g_abort_on_error.exchange(on ? 1 : 0); }
const char* malus_last_error(void) { return g_last_error.c_str(); }
void malus_clear_error(void) { g_last_error.clear(); }

void malus_init(void) { API_TRY ensure_init(); API_CATCH() }

int64_t tensor_alloc_gpu(int32_t dtype, const size_t* shape, size_t ndim, const void* data) {
  API_TRY
  if (dtype != F32 && dtype != I32 && dtype != I64)
    fail("malus: unsupported dtype tag %d; supported: f32, i32, i64", dtype);
  TensorBuffer* t = alloc_tensor(dtype, shape, (int)ndim);
  if (data && t->len) {
    upload(t->data(), data, t->bytes());
    t->write_seq = enqueue_mark("tensor_alloc_gpu");
  }
  return H(t);
  API_CATCH(0)
}

int64_t tensor_alloc_zeros_gpu(const size_t* shape, size_t ndim) {
  API_TRY
  TensorBuffer* t = alloc_tensor(F32, shape, (int)ndim);
  k::fill(t->f32(), 0.0f, t->len, stream());  // fill kernel (graph-capture safe)
  t->write_seq = enqueue_mark("zeros");
  return H(t);
  API_CATCH(0)
}

int64_t tensor_alloc_ones_gpu(const size_t* shape, size_t ndim) {
  API_TRY
  TensorBuffer* t = alloc_tensor(F32, shape, (int)ndim);
  k::fill(t->f32(), 1.0f, t->len, stream());
  t->write_seq = enqueue_mark("ones");
  return H(t);
  API_CATCH(0)
}

void tensor_retain(int64_t h) { API_TRY retain(T(h)); API_CATCH() }
void tensor_release(int64_t h) { API_TRY release(T(h)); API_CATCH() }
void tensor_free(int64_t h) { API_TRY release(T(h)); API_CATCH() }

int64_t tensor_len(int64_t h) { return (int64_t)T(h)->len; }
int64_t tensor_ndim(int64_t h) { return (int64_t)T(h)->ndim; }
int64_t tensor_dim(int64_t h, int64_t i) {
  API_TRY
  TensorBuffer* t = T(h);
  int64_t idx = i < 0 ? i + t->ndim : i;
  if (idx < 0 || idx >= t->ndim) fail("malus: tensor_dim index %lld out of range for rank-%d tensor", (long long)i, t->ndim);
  return (int64_t)t->shape[idx];
  API_CATCH(0)
}
int32_t malus_tensor_dtype(int64_t h) { return T(h)->dtype; }
void malus_tensor_shape(int64_t h, size_t* out) {
  for (int i = 0; i < T(h)->ndim; ++i) out[i] = T(h)->shape[i];
}

void tensor_print(int64_t h) {
  API_TRY
  if (h == 0) { fputs("[]", stdout); return; }
  TensorBuffer* t = T(h);
  std::vector<char> host(t->bytes() + 8);
  download(host.data(), t, t->bytes());
  if (t->dtype == I32) {
    print_nd(reinterpret_cast<const int32_t*>(host.data()), t->shape, t->ndim, 0,
             [](int32_t v) { return std::to_string(v); });
  } else if (t->dtype == I64) {
    print_nd(reinterpret_cast<const int64_t*>(host.data()), t->shape, t->ndim, 0,
             [](int64_t v) { return std::to_string(v); });
  } else {
    print_nd(reinterpret_cast<const float*>(host.data()), t->shape, t->ndim, 0, rust_f32);
  }
  fflush(stdout);
  API_CATCH()
}

size_t malus_format_f32(float v, char* buf, size_t cap) {
  std::string s = rust_f32(v);
  if (cap) { strncpy(buf, s.c_str(), cap - 1); buf[cap - 1] = 0; }
  return s.size();
}

float malus_tensor_get_f32(int64_t h, int64_t idx) {
  API_TRY
  TensorBuffer* t = T(h);
  if (idx < 0 || (size_t)idx >= t->len) fail("malus: tensor_get_f32 index %lld out of range for len %zu", (long long)idx, t->len);
  materialize_upper_tiles(t);
  flush_if_pending(t);
  float v;
  MALUS_HIP(hipMemcpyAsync(&v, t->f32() + idx, sizeof(float), hipMemcpyDeviceToHost, stream()));
  MALUS_HIP(hipStreamSynchronize(stream()));
  return v;
  API_CATCH(0.0f)
}

// Copy a tensor's contents to host memory (flushes pending writes).
void malus_tensor_read(int64_t h, void* dst, size_t bytes) {
  API_TRY
  TensorBuffer* t = T(h);
  if (bytes > t->bytes()) fail("malus: tensor_read of %zu bytes from a %zu-byte tensor", bytes, t->bytes());
  download(dst, t, bytes);
  API_CATCH()
}

// Overwrite a tensor's contents from host memory (stream-ordered).
// The device address of a tensor's storage (NULL for a shape-only handle).
void* malus_tensor_device_ptr(int64_t h) {
  TensorBuffer* t = T(h);
  return t && t->st ? t->st->ptr : nullptr;
}

void malus_tensor_write(int64_t h, const void* src, size_t bytes) {
  API_TRY
  TensorBuffer* t = T(h);
  if (bytes > t->bytes()) fail("malus: tensor_write of %zu bytes into a %zu-byte tensor", bytes, t->bytes());
  materialize_upper_tiles(t);  // a partial write keeps the rest
  upload(t->data(), src, bytes);
  t->st->causal_t = 0;
  t->st->causal_mask_t = 0;
  t->write_seq = enqueue_mark("tensor_write");
  API_CATCH()
}

void gpu_barrier(void) { API_TRY sync_all(); API_CATCH() }

void malus_flush_if_pending(int64_t h) { API_TRY flush_if_pending(T(h)); API_CATCH() }
int tensor_is_pending(int64_t h) { return T(h)->write_seq > ctx().completed.load() ? 1 : 0; }

int64_t tensor_reshape(int64_t h, const size_t* dims, size_t ndim) {
  API_TRY
  TensorBuffer* t = T(h);
  size_t n = 1;
  for (size_t i = 0; i < ndim; ++i) n *= dims[i];
  if (n != t->len) {
    TensorBuffer tmp;
    tmp.ndim = (int)ndim;
    for (size_t i = 0; i < ndim && i < (size_t)kMaxRank; ++i) tmp.shape[i] = dims[i];
    fail("malus: reshape element count mismatch: input shape %s has %zu elements, target shape %s would have %zu",
         shape_str(t).c_str(), t->len, shape_str(&tmp).c_str(), n);
  }
  return H(make_alias(t, dims, (int)ndim));
  API_CATCH(0)
}

int64_t tensor_causal_mask(int64_t tsz) {
  API_TRY
  size_t sh[2] = {(size_t)tsz, (size_t)tsz};
  TensorBuffer* t = alloc_tensor(F32, sh, 2);
  k::causal_mask(t->f32(), (size_t)tsz, stream());
  t->st->causal_mask_t = (uint32_t)tsz;
  t->write_seq = enqueue_mark("causal_mask");
  return H(t);
  API_CATCH(0)
}

int64_t tensor_randn(const size_t* shape, size_t ndim) {
  API_TRY
  // metal.rs:1720-1740: host Philox keyed by the per-thread call counter,
  // Box-Muller in f64, placed on the device.
  size_t n = 1;
  for (size_t i = 0; i < ndim; ++i) n *= shape[i];
  uint64_t call = rng_next_call();
  uint32_t key[2] = {(uint32_t)call, (uint32_t)(call >> 32)};
  std::vector<float> data(n ? n : 1);
  const double two_pi = 2.0 * 3.14159265358979311599796346854;
  for (size_t k = 0; k < (n + 1) / 2; ++k) {
    uint32_t ctr[4] = {(uint32_t)k, (uint32_t)((uint64_t)k >> 32), 0u, 0u}, r[4];
    philox4x32_10(ctr, key, r);
    double u1 = ((double)r[0] + 0.5) / 4294967296.0;
    double u2 = ((double)r[1] + 0.5) / 4294967296.0;
    double mag = std::sqrt(-2.0 * std::log(u1));
    data[2 * k] = (float)(mag * std::cos(two_pi * u2));
    if (2 * k + 1 < n) data[2 * k + 1] = (float)(mag * std::sin(two_pi * u2));
  }
  return tensor_alloc_gpu(F32, shape, ndim, data.data());
  API_CATCH(0)
}

float malus_rand_uniform(void) {
  uint64_t call = rng_next_call();
  uint32_t key[2] = {(uint32_t)call, (uint32_t)(call >> 32)}, ctr[4] = {0, 0, 0, 0}, r[4];
  philox4x32_10(ctr, key, r);
  return (float)((double)r[0] / 4294967296.0);
}

int64_t malus_rand_int(int64_t n) {
  API_TRY
  if (n <= 0) fail("malus: rand_int bound must be positive, got %lld", (long long)n);
  uint64_t call = rng_next_call();
  uint32_t key[2] = {(uint32_t)call, (uint32_t)(call >> 32)}, ctr[4] = {1, 0, 0, 0}, r[4];
  philox4x32_10(ctr, key, r);
  return (int64_t)((uint64_t)r[0] % (uint64_t)n);
  API_CATCH(0)
}

// ---- the device-side data path (no reference counterpart) ------------------
// randn with the reference's stream (metal.rs:1720-1740), generated on the
// device: the same Philox words; the same f64 Box-Muller.
int64_t malus_randn_device(const size_t* shape, size_t ndim) {
  API_TRY
  TensorBuffer* t = alloc_tensor(F32, shape, (int)ndim);
  const uint64_t call = rng_next_call();
  k::randn(t->f32(), t->len, call, stream());
  t->write_seq = enqueue_mark("randn_device");
  return H(t);
  API_CATCH(0)
}

// i.i.d. token ids on the device: out[i] = rand_int(vocab) with call index
// call + i, the ids the host builtin's loop draws (metal.rs:1741-1759).  A new
// [n] i32 tensor.
int64_t malus_rand_tokens_device(uint64_t call, size_t n, int64_t vocab) {
  API_TRY
  if (vocab < 1 || vocab > INT32_MAX) fail("malus: rand_tokens: vocab %lld out of range", (long long)vocab);
  const size_t sh[1] = {n};
  TensorBuffer* t = alloc_tensor(I32, sh, 1);
  k::rand_tokens(t->i32(), nullptr, n, nullptr, call, 0, (uint32_t)vocab, stream());
  t->write_seq = enqueue_mark("rand_tokens");
  return H(t);
  API_CATCH(0)
}

// The batch of nanogpt_modular.ml:170-177 built on the device from a
// device-resident i32 token stream `data`: for b in 0..B, start =
// rand_int(len(data) - T - 1) (one RNG call each, as the host loop makes
// them), x[b*T + t] = data[start + t], y[b*T + t] = data[start + t + 1].
// x and y are new [B*T] i32 tensors.  starts_out (optional, host int32[B])
// receives the starts, which costs a device read.
void malus_batch_windows(int64_t data, int64_t B, int64_t Tn, int64_t* x_out, int64_t* y_out, int32_t* starts_out) {
  API_TRY
  TensorBuffer* d = T(data);
  if (d->dtype != I32 || d->ndim != 1) fail("malus: batch_windows: data must be a 1-D i32 tensor, got %s", shape_str(d).c_str());
  if (B <= 0 || Tn <= 0 || B > 65535) fail("malus: batch_windows: bad batch %lld x %lld", (long long)B, (long long)Tn);
  if ((int64_t)d->len < Tn + 2) fail("malus: batch_windows: %zu tokens cannot hold a window of %lld + 1", d->len, (long long)Tn);
  if (!x_out || !y_out) fail("malus: batch_windows: null output");
  const uint64_t range = (uint64_t)(d->len - (size_t)Tn - 1);
  const uint64_t call0 = t_rng_calls;
  t_rng_calls += (uint64_t)B;
  const size_t sh[1] = {(size_t)(B * Tn)};
  TensorBuffer *x = alloc_tensor(I32, sh, 1), *y = alloc_tensor(I32, sh, 1);
  size_t bucket = 0;
  int32_t* starts = starts_out ? static_cast<int32_t*>(pool_alloc((size_t)B * sizeof(int32_t), &bucket)) : nullptr;
  k::batch_windows(d->i32(), x->i32(), y->i32(), (size_t)B, (size_t)Tn, call0, range, starts, stream());
  x->write_seq = y->write_seq = enqueue_mark("batch_windows");
  if (starts) {
    MALUS_HIP(hipMemcpyAsync(starts_out, starts, (size_t)B * sizeof(int32_t), hipMemcpyDeviceToHost, stream()));
    MALUS_HIP(hipStreamSynchronize(stream()));
    pool_free(starts, bucket);
  }
  *x_out = H(x);
  *y_out = H(y);
  API_CATCH()
}

uint64_t malus_rng_get_counter(void) { return t_rng_calls; }
void malus_rng_set_counter(uint64_t v) { t_rng_calls = v; }

// ---- Buffer<i32> (buffer.rs:1-50) -------------------------------------------
struct BufferData { size_t len; std::vector<int32_t> data; };

int64_t malus_buffer_i32(int64_t len) {
  auto* b = new BufferData{(size_t)len, std::vector<int32_t>((size_t)len, 0)};
  return reinterpret_cast<int64_t>(b);
}
int64_t malus_buffer_get_i32(int64_t h, int64_t i) {
  API_TRY
  auto* b = reinterpret_cast<BufferData*>(h);
  if (i < 0 || (size_t)i >= b->len) fail("malus: buffer index %lld out of range for len %zu", (long long)i, b->len);
  return b->data[(size_t)i];
  API_CATCH(0)
}
void malus_buffer_set_i32(int64_t h, int64_t i, int64_t v) {
  API_TRY
  auto* b = reinterpret_cast<BufferData*>(h);
  if (i < 0 || (size_t)i >= b->len) fail("malus: buffer index %lld out of range for len %zu", (long long)i, b->len);
  b->data[(size_t)i] = (int32_t)v;
  API_CATCH()
}
void malus_buffer_free(int64_t h) {
  if (!h) return;
  delete reinterpret_cast<BufferData*>(h);
}
int64_t malus_buffer_freeze_i32(int64_t h) {
  auto* b = reinterpret_cast<BufferData*>(h);
  size_t sh[1] = {b->len};
  return tensor_alloc_gpu(I32, sh, 1, b->data.data());
}

// ---- bench timer (bench.rs:1-76, ADR-0038) ----------------------------------
static std::atomic<bool> g_bench_on{false};
static std::chrono::steady_clock::time_point g_step_start;
static bool g_step_open = false;
static std::vector<double> g_step_ms;

void bench_enable(void) { g_bench_on = true; }
void bench_reset(void) {
  g_bench_on = false;
  g_step_open = false;
  g_step_ms.clear();
}
void bench_step_begin(void) {
  if (!g_bench_on) return;
  g_step_start = std::chrono::steady_clock::now();
  g_step_open = true;
}
void bench_step_end(void) {
  if (!g_bench_on) return;
  gpu_barrier();  // flush inside the timed region (bench.rs:29-38)
  if (g_step_open) {
    g_step_ms.push_back(std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - g_step_start).count());
    g_step_open = false;
  }
}
// Warm median (skip 3; even count -> mean of the middle two), bench.rs:51-70.
int bench_report(double* median_ms, double* min_ms, double* max_ms, int64_t* warm_steps) {
  const size_t warmup = 3;
  if (g_step_ms.size() <= warmup) return 0;
  std::vector<double> w(g_step_ms.begin() + warmup, g_step_ms.end());
  std::sort(w.begin(), w.end());
  size_t n = w.size();
  *median_ms = n % 2 ? w[n / 2] : (w[n / 2 - 1] + w[n / 2]) / 2.0;
  *min_ms = w[0];
  *max_ms = w[n - 1];
  *warm_steps = (int64_t)n;
  return 1;
}
void malus_bench_record(double ms) { g_step_ms.push_back(ms); }

// ---- counters ----------------------------------------------------------------
int64_t malus_cpu_compute_count(void) { return 0; }  // the product has no CPU compute path
void malus_cpu_compute_reset(void) {}
void malus_rc_counts(int64_t* out3) { out3[0] = g_retain; out3[1] = g_release; out3[2] = g_alloc; }
void malus_rc_reset(void) { g_retain = 0; g_release = 0; g_alloc = 0; }

void malus_record_diff(float v) {
  float a = std::fabs(v);
  uint32_t bits;
  memcpy(&bits, &a, 4);
  uint32_t cur = g_gradcheck_bits.load();
  while (true) {
    float cf;
    memcpy(&cf, &cur, 4);
    if (a <= cf) return;
    if (g_gradcheck_bits.compare_exchange_weak(cur, bits)) return;
  }
}
float malus_gradcheck_max_diff(void) {
  uint32_t b = g_gradcheck_bits.load();
  float f;
  memcpy(&f, &b, 4);
  return f;
}
void malus_gradcheck_reset(void) { g_gradcheck_bits = 0; }

// ---- pool stats ---------------------------------------------------------------
void malus_pool_stats(int64_t* out4) {
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.pool.mu);
  out4[0] = c.pool.hits;
  out4[1] = c.pool.misses;
  out4[2] = c.pool.pooled_bytes;
  out4[3] = c.pool.peak_bytes;
}
int64_t malus_pool_live_bytes(void) {
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.pool.mu);
  return c.pool.live_bytes;
}
size_t malus_pool_buckets(size_t* sizes, size_t* counts, size_t cap) {
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.pool.mu);
  std::vector<std::pair<size_t, size_t>> v;
  for (auto& kv : c.pool.free_lists) v.push_back({kv.first, kv.second.size()});
  std::sort(v.begin(), v.end());
  for (size_t i = 0; i < v.size() && i < cap; ++i) { sizes[i] = v[i].first; counts[i] = v[i].second; }
  return v.size();
}
void malus_pool_reset(void) {
  API_TRY
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.pool.mu);
  trim_pool(c);
  c.pool.hits = c.pool.misses = 0;
  c.pool.pooled_bytes = 0;
  c.pool.peak_bytes = c.pool.live_bytes;
  API_CATCH()
}
void malus_set_mem_budget(int64_t bytes) { ctx().budget = bytes < 0 ? -1 : bytes; }
void malus_fail_alloc_after(int64_t n) { ctx().fail_alloc_after = n < 0 ? -1 : n; }
size_t malus_alloc_histogram(size_t* sizes, uint64_t* counts, size_t cap) {
  Context& c = ctx();
  std::lock_guard<std::mutex> lk(c.pool.mu);
  size_t i = 0;
  for (auto& kv : c.pool.histogram) {
    if (i < cap) { sizes[i] = kv.first; counts[i] = kv.second; }
    ++i;
  }
  return c.pool.histogram.size();
}

// ---- per-kernel timing ----------------------------------------------------------
void malus_ktimer_enable(int on) { g_ktimer_on = on != 0; }
// Sum the recorded launches of one class (all classes when cls is null);
// returns the number of launches and clears them.
int64_t malus_ktimer_collect(const char* cls, double* total_ms, double* total_units) {
  API_TRY
  sync_all();
  std::lock_guard<std::mutex> lk(g_ktimer_mu);
  double ms = 0, units = 0;
  int64_t n = 0;
  std::vector<KTimer*> keep;
  for (KTimer* t : g_ktimers) {
    if (!cls || strcmp(cls, t->cls) == 0) {
      float e = 0;
      MALUS_HIP(hipEventElapsedTime(&e, t->e0, t->e1));
      ms += e;
      units += t->units;
      ++n;
      g_ktimer_spare.push_back(t);
    } else {
      keep.push_back(t);
    }
  }
  g_ktimers.swap(keep);
  if (total_ms) *total_ms = ms;
  if (total_units) *total_units = units;
  return n;
  API_CATCH(0)
}

// Device info for reports.
int malus_device_info(char* name, size_t cap, int* cus, int* clock_khz) {
  API_TRY
  hipDeviceProp_t p;
  MALUS_HIP(hipGetDeviceProperties(&p, ctx().device));
  if (cap) { strncpy(name, p.gcnArchName, cap - 1); name[cap - 1] = 0; }
  *cus = p.multiProcessorCount;
  *clock_khz = p.clockRate;
  return 1;
  API_CATCH(0)
}

}  // extern "C"
