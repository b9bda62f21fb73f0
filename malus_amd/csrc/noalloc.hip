// The allocation-free entry point: the axis reduction of
// malus_std_reduce_fwd on caller-owned device buffers, with its temporaries
// (split partials, the variance's mean) in a fixed device array of this
// library instead of the pool.  For callers that cannot allocate device
// memory (HIP graph capture, serving loops, harnesses that forbid hipMalloc).
//
// `scratch` is one file-scope device array: every GPU the library runs on
// holds its own copy (kNoAllocScratchBytes) until the process ends.  Host
// code never passes the array's name to a kernel (on the host it only names
// a stand-in symbol): its device address is taken with hipGetSymbolAddress
// once per device at library set-up, with that device current, and only
// that address is used afterwards.
//
// Every call on one GPU shares the array and it keeps the last call's
// contents.  The kernels write every partial before they read it, so nothing
// in it needs to start at zero.  Calls are enqueued on the library's stream,
// so calls from one host thread are ordered; calls that overlap (from
// several host threads) race on the array.
#include <cstdint>
#include <mutex>

#include "api.h"
#include "common.h"

namespace {

constexpr size_t kNoAllocScratchBytes = size_t(4) << 20;  // 4 MiB per device
constexpr size_t kNoAllocScratchFloats = kNoAllocScratchBytes / sizeof(float);
constexpr int kMaxDevices = 64;

static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

std::mutex g_mu;
float* g_scratch_ptr[kMaxDevices] = {};  // device address of `scratch` per device

}  // namespace

namespace malus {

// Set-up (called by the library's init, with the library's device current):
// the device address of this device's copy of `scratch`.
void noalloc_init_device(int device) {
  if (device < 0 || device >= kMaxDevices) fail("malus: device %d out of range for the no-alloc scratch table", device);
  std::lock_guard<std::mutex> lk(g_mu);
  if (g_scratch_ptr[device]) return;
  void* p = nullptr;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p)
    fail("malus: hipGetSymbolAddress(scratch) failed on device %d: %s", device, hipGetErrorString(e));
  g_scratch_ptr[device] = static_cast<float*>(p);
}

}  // namespace malus

extern "C" {

int malus_std_reduce_noalloc(int32_t op, const float* x, const size_t* shape, size_t ndim, int64_t axis, float* out) {
  API_TRY
  using namespace malus;
  int dev = -1;
  MALUS_HIP(hipGetDevice(&dev));
  float* base = (dev >= 0 && dev < kMaxDevices) ? g_scratch_ptr[dev] : nullptr;
  if (!base) fail("malus: reduce_noalloc: call malus_init() on device %d first (it sets up the scratch array)", dev);
  if (op < 0 || op > 3) fail("malus: reduce_noalloc: bad reduction op %d", (int)op);
  if (!shape || ndim == 0 || ndim > (size_t)kMaxRank) fail("malus: reduce_noalloc: rank %zu not in 1..%d", ndim, kMaxRank);
  const int64_t nd = (int64_t)ndim;
  if (axis < -nd || axis >= nd) fail("malus: reduce_noalloc: axis %lld out of range for rank %zu", (long long)axis, ndim);
  const size_t ax = (size_t)(axis < 0 ? axis + nd : axis);
  size_t outer = 1, inner = 1;
  for (size_t i = 0; i < ax; ++i) outer *= shape[i];
  for (size_t i = ax + 1; i < ndim; ++i) inner *= shape[i];
  const size_t len = shape[ax];
  if (outer * inner == 0) return 0;
  if (!x || !out) fail("malus: reduce_noalloc: null input or output pointer");
  const size_t need = k::reduce_axis_scratch_floats(op, x, out, outer, len, inner);
  if (need > kNoAllocScratchFloats)
    fail("malus: reduce_noalloc: this reduction needs %zu bytes of scratch, more than the %zu-byte array",
         need * sizeof(float), kNoAllocScratchBytes);
  k::reduce_axis_scratch(op, x, out, outer, len, inner, base, kNoAllocScratchFloats, stream());
  enqueue_mark("reduce_noalloc");
  return 0;
  API_CATCH(-1)
}

}  // extern "C"
