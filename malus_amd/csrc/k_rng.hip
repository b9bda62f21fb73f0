// Device-side random streams and batch construction (the "device-side data
// path": no host Philox loop, no host token buffers, no per-step upload).
//
// Philox4x32-10 is the published Random123 generator (the round constants
// below are its published multipliers and Weyl increments); the counter and
// key use is the reference's (metal.rs:1713-1759): key = the per-thread call
// index, counter = [pair index, 0, 0, 0] for randn, [1, 0, 0, 0] for
// rand_int.  The integer words are bit-exact with the host generator;
// randn's Box-Muller runs in f64 as the host's does.
#include "common.h"

namespace malus {
namespace k {
namespace {

__device__ __forceinline__ void philox(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0, uint32_t k1,
                                       uint32_t out[4]) {
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)c0 * 0xD2511F53u, p1 = (uint64_t)c2 * 0xCD9E8D57u;
    const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0, n1 = (uint32_t)p1;
    const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1, n3 = (uint32_t)p0;
    c0 = n0;
    c1 = n1;
    c2 = n2;
    c3 = n3;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  out[0] = c0;
  out[1] = c1;
  out[2] = c2;
  out[3] = c3;
}

// pair k -> out[2k], out[2k+1] (the second one only while in range)
__global__ __launch_bounds__(256) void k_randn(float* __restrict__ out, size_t n, uint32_t key0, uint32_t key1) {
  const size_t pairs = (n + 1) / 2, stride = (size_t)gridDim.x * blockDim.x;
  const double two_pi = 2.0 * 3.14159265358979311599796346854;
  for (size_t k = (size_t)blockIdx.x * blockDim.x + threadIdx.x; k < pairs; k += stride) {
    uint32_t r[4];
    philox((uint32_t)k, (uint32_t)((uint64_t)k >> 32), 0u, 0u, key0, key1, r);
    const double u1 = ((double)r[0] + 0.5) / 4294967296.0;
    const double u2 = ((double)r[1] + 0.5) / 4294967296.0;
    const double mag = sqrt(-2.0 * log(u1));
    out[2 * k] = (float)(mag * cos(two_pi * u2));
    if (2 * k + 1 < n) out[2 * k + 1] = (float)(mag * sin(two_pi * u2));
  }
}

// Sequence b of the batch starts at rand_int(range) drawn with call index
// call0 + b; x[b, t] = data[start + t], y[b, t] = data[start + t + 1].
__global__ __launch_bounds__(256) void k_batch_windows(const int32_t* __restrict__ data, int32_t* __restrict__ x,
                                                       int32_t* __restrict__ y, uint32_t B, uint32_t T, uint64_t call0,
                                                       uint64_t range, int32_t* __restrict__ starts) {
  const uint32_t b = blockIdx.x;
  if (b >= B) return;
  __shared__ uint64_t start;
  if (threadIdx.x == 0) {
    const uint64_t call = call0 + b;
    uint32_t r[4];
    philox(1u, 0u, 0u, 0u, (uint32_t)call, (uint32_t)(call >> 32), r);
    start = (uint64_t)r[0] % range;
    if (starts) starts[b] = (int32_t)start;
  }
  __syncthreads();
  const size_t base = (size_t)b * T;
  for (uint32_t t = threadIdx.x; t < T; t += blockDim.x) {
    x[base + t] = data[start + t];
    y[base + t] = data[start + t + 1];
  }
}

// i.i.d. token ids: x[i] = rand_int(vocab) with call index cx + i, y[i]
// the same with cy + i (the `rand_int` builtin: counter [1, 0, 0, 0], key =
// the call index; the word's remainder by vocab).  The two call indices come
// from `calls` in device memory when it is given (a captured step reads each
// replay's own), else from cx and cy.  y may be null (x only).
__global__ __launch_bounds__(256) void k_rand_tokens(int32_t* __restrict__ x, int32_t* __restrict__ y, size_t n,
                                                     const uint64_t* __restrict__ calls, uint64_t cx, uint64_t cy,
                                                     uint32_t vocab) {
  if (calls) {
    cx = calls[0];
    cy = calls[1];
  }
  const size_t stride = (size_t)gridDim.x * blockDim.x, total = y ? 2 * n : n;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const bool second = i >= n;
    const uint64_t call = (second ? cy : cx) + (second ? i - n : i);
    uint32_t r[4];
    philox(1u, 0u, 0u, 0u, (uint32_t)call, (uint32_t)(call >> 32), r);
    (second ? y : x)[second ? i - n : i] = (int32_t)(r[0] % vocab);
  }
}

}  // namespace

void rand_tokens(int32_t* x, int32_t* y, size_t n, const uint64_t* calls, uint64_t cx, uint64_t cy, uint32_t vocab,
                 hipStream_t s) {
  if (!n) return;
  size_t blocks = ((y ? 2 * n : n) + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  k_rand_tokens<<<(unsigned)blocks, 256, 0, s>>>(x, y, n, calls, cx, cy, vocab);
  MALUS_HIP(hipGetLastError());
}

void randn(float* out, size_t n, uint64_t call, hipStream_t s) {
  if (!n) return;
  size_t blocks = ((n + 1) / 2 + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  k_randn<<<(unsigned)blocks, 256, 0, s>>>(out, n, (uint32_t)call, (uint32_t)(call >> 32));
  MALUS_HIP(hipGetLastError());
}

void batch_windows(const int32_t* data, int32_t* x, int32_t* y, size_t B, size_t T, uint64_t call0, uint64_t range,
                   int32_t* starts, hipStream_t s) {
  if (!B || !T) return;
  k_batch_windows<<<(unsigned)B, 256, 0, s>>>(data, x, y, (uint32_t)B, (uint32_t)T, call0, range, starts);
  MALUS_HIP(hipGetLastError());
}

}  // namespace k
}  // namespace malus
