// Axis reductions (sum / mean / max / population variance) over any axis
// length — the reference's single-threadgroup kernels cap the axis at 1024
// (reduce_sum.ml:13); these do not.  A contiguous tensor is viewed as
// [outer, axis, inner]:
//   inner == 1 : row reduction, one wave64 per row (shuffle tree), or a
//                two-stage split when rows are long and few;
//   inner  > 1 : column reduction, coalesced over inner, the axis split into
//                chunks whose partials are combined in chunk order.
// Every order is fixed, so results are run-to-run deterministic.
#include "common.h"

namespace malus {
namespace k {
namespace {

constexpr int kWave = 64;

template <int OP>
__device__ __forceinline__ float rinit() { return OP == R_MAX ? -INFINITY : 0.0f; }

template <int OP>
__device__ __forceinline__ float rcomb(float a, float b) { return OP == R_MAX ? fmaxf(a, b) : a + b; }

// element transform: VAR accumulates (x - mean)^2; others use x.
template <int OP>
__device__ __forceinline__ float rload(float x, float mean) {
  if constexpr (OP == R_VAR) { float d = x - mean; return d * d; }
  else return x;
}

template <int OP>
__device__ __forceinline__ float wave_reduce(float v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v = rcomb<OP>(v, __shfl_xor(v, off, kWave));
  return v;
}

// Finalize: MEAN and VAR divide the accumulated sum by the axis length.
template <int OP>
__device__ __forceinline__ float rfinal(float s, uint32_t count) {
  if constexpr (OP == R_MEAN || OP == R_VAR) return s / (float)count;
  else return s;
}

// One wave per row; rows are contiguous of length `axis`.  `mean` (VAR
// only) holds one value per row.  FINAL divides by `count`.
template <int OP, bool VEC>
__global__ __launch_bounds__(256) void k_row_wave(const float* __restrict__ x, const float* __restrict__ mean,
                                                  float* __restrict__ out, size_t rows, uint32_t axis, uint32_t count,
                                                  bool finalize) {
  const size_t row = (size_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (row >= rows) return;
  const float* xr = x + row * axis;
  const float mu = (OP == R_VAR) ? mean[row] : 0.0f;
  float acc = rinit<OP>();
  if (VEC) {
    const float4* x4 = reinterpret_cast<const float4*>(xr);
    const uint32_t n4 = axis / 4;
    for (uint32_t i = lane; i < n4; i += kWave) {
      float4 v = x4[i];
      acc = rcomb<OP>(acc, rload<OP>(v.x, mu));
      acc = rcomb<OP>(acc, rload<OP>(v.y, mu));
      acc = rcomb<OP>(acc, rload<OP>(v.z, mu));
      acc = rcomb<OP>(acc, rload<OP>(v.w, mu));
    }
  } else {
    for (uint32_t i = lane; i < axis; i += kWave) acc = rcomb<OP>(acc, rload<OP>(xr[i], mu));
  }
  acc = wave_reduce<OP>(acc);
  if (lane == 0) out[row] = finalize ? rfinal<OP>(acc, count) : acc;
}

// Split long rows: block (row, split) reduces [split*chunk, ...) of the row
// into partial[row * nsplit + split].
template <int OP>
__global__ __launch_bounds__(256) void k_row_split(const float* __restrict__ x, const float* __restrict__ mean,
                                                   float* __restrict__ partial, size_t rows, size_t axis,
                                                   uint32_t nsplit, size_t chunk) {
  __shared__ float red[256 / kWave];
  const size_t bid = blockIdx.x;
  const size_t row = bid / nsplit;
  const uint32_t sp = (uint32_t)(bid % nsplit);
  const float* xr = x + row * axis;
  const float mu = (OP == R_VAR) ? mean[row] : 0.0f;
  size_t beg = sp * chunk, end = beg + chunk < axis ? beg + chunk : axis;
  float acc = rinit<OP>();
  // chunk is a multiple of 4 and rows are 16-byte aligned when axis % 4 == 0
  if ((axis & 3) == 0) {
    const float4* x4 = reinterpret_cast<const float4*>(xr);
    for (size_t i = beg / 4 + threadIdx.x; i < end / 4; i += blockDim.x) {
      float4 v = x4[i];
      acc = rcomb<OP>(acc, rload<OP>(v.x, mu));
      acc = rcomb<OP>(acc, rload<OP>(v.y, mu));
      acc = rcomb<OP>(acc, rload<OP>(v.z, mu));
      acc = rcomb<OP>(acc, rload<OP>(v.w, mu));
    }
  } else {
    for (size_t i = beg + threadIdx.x; i < end; i += blockDim.x) acc = rcomb<OP>(acc, rload<OP>(xr[i], mu));
  }
  acc = wave_reduce<OP>(acc);
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float r = red[0];
    for (int w = 1; w < (int)(blockDim.x / kWave); ++w) r = rcomb<OP>(r, red[w]);
    partial[row * nsplit + sp] = r;
    (void)rows;
  }
}

// Column reduction: out[o, i] over a = 0..axis-1 of x[o, a, i].  Thread
// handles one column i for the axis chunk [sp*chunk, ...).  nsplit == 1
// writes the finalized value; otherwise partial[(o * nsplit + sp) * inner + i].
template <int OP>
__global__ __launch_bounds__(256) void k_col(const float* __restrict__ x, const float* __restrict__ mean,
                                             float* __restrict__ dst, size_t outer, size_t axis, size_t inner,
                                             uint32_t nsplit, size_t chunk, uint32_t col_blocks, bool finalize) {
  size_t bid = blockIdx.x;
  const uint32_t cb = (uint32_t)(bid % col_blocks);
  bid /= col_blocks;
  const uint32_t sp = (uint32_t)(bid % nsplit);
  const size_t o = bid / nsplit;
  const size_t i = (size_t)cb * blockDim.x + threadIdx.x;
  if (i >= inner || o >= outer) return;
  const float mu = (OP == R_VAR) ? mean[o * inner + i] : 0.0f;
  size_t beg = sp * chunk, end = beg + chunk < axis ? beg + chunk : axis;
  const float* xp = x + o * axis * inner + i;
  float acc = rinit<OP>();
  for (size_t a = beg; a < end; ++a) acc = rcomb<OP>(acc, rload<OP>(xp[a * inner], mu));
  if (nsplit == 1) dst[o * inner + i] = finalize ? rfinal<OP>(acc, (uint32_t)axis) : acc;
  else dst[(o * nsplit + sp) * inner + i] = acc;
}

// Combine column partials.  Block (x, o) owns kCombCols consecutive columns;
// its 256 threads form 16 split groups, group g summing splits g, g+16, ...
// in order (each group's loads of one split row are contiguous), then the 16
// group sums are folded in group order.  Fixed order, so deterministic.
constexpr int kCombCols = 16;
template <int OP>
__global__ __launch_bounds__(256) void k_col_combine(const float* __restrict__ partial, float* __restrict__ out,
                                                     uint32_t nsplit, size_t inner, uint32_t count) {
  constexpr int G = 256 / kCombCols;
  __shared__ float red[G][kCombCols + 1];
  const int lc = threadIdx.x % kCombCols, g = threadIdx.x / kCombCols;
  const size_t o = blockIdx.y;
  const size_t i = (size_t)blockIdx.x * kCombCols + lc;
  float acc = rinit<OP>();
  if (i < inner) {
    const float* p = partial + o * nsplit * inner + i;
    for (uint32_t s = g; s < nsplit; s += G) acc = rcomb<OP>(acc, p[(size_t)s * inner]);
  }
  red[g][lc] = acc;
  __syncthreads();
  if (g == 0 && i < inner) {
    float r = red[0][lc];
#pragma unroll
    for (int w = 1; w < G; ++w) r = rcomb<OP>(r, red[w][lc]);
    out[o * inner + i] = rfinal<OP>(r, count);
  }
}

__global__ __launch_bounds__(256) void k_expand_axis(const float* __restrict__ small, float* __restrict__ out,
                                                     size_t n, size_t axis, size_t inner) {
  // reduce_bwd.ml:10-18: out[o, a, i] = small[o, i]
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t f = (size_t)blockIdx.x * blockDim.x + threadIdx.x; f < n; f += stride) {
    size_t o = f / (axis * inner), iv = f % inner;
    out[f] = small[o * inner + iv];
  }
}

template <int OP>
void reduce_impl(const float* x, const float* mean, float* out, size_t outer, size_t axis, size_t inner, hipStream_t s) {
  const size_t n_out = outer * inner;
  if (n_out == 0) return;
  if (axis == 0) {  // empty reduction: sum/mean identities (mean/var of nothing -> NaN like 0/0)
    if (OP == R_MAX) fill(out, -INFINITY, n_out, s);
    else if (OP == R_SUM) fill(out, 0.0f, n_out, s);
    else fill(out, NAN, n_out, s);
    return;
  }
  if (inner == 1) {
    const size_t rows = outer;
    // Long rows with few of them: split each row across blocks.
    if (axis >= 16384 && rows < 2048) {
      size_t want_blocks = 2048;
      uint32_t nsplit = (uint32_t)((want_blocks + rows - 1) / rows);
      size_t chunk = (axis + nsplit - 1) / nsplit;
      chunk = (chunk + 1023) / 1024 * 1024;  // multiple of 4, float4-friendly
      nsplit = (uint32_t)((axis + chunk - 1) / chunk);
      size_t bucket;
      float* partial = static_cast<float*>(pool_alloc(rows * nsplit * sizeof(float), &bucket));
      k_row_split<OP><<<(unsigned)(rows * nsplit), 256, 0, s>>>(x, mean, partial, rows, axis, nsplit, chunk);
      MALUS_HIP(hipGetLastError());
      // combine partials of each row with one wave per row, then finalize
      // (MEAN/VAR: the partials are plain sums, so combine them with SUM)
      constexpr int COMB = (OP == R_MAX) ? R_MAX : R_SUM;
      k_row_wave<COMB, false><<<(unsigned)((rows + 3) / 4), 256, 0, s>>>(partial, nullptr, out, rows, nsplit, nsplit, false);
      MALUS_HIP(hipGetLastError());
      if (OP == R_MEAN || OP == R_VAR) {
        // divide in place by the axis length
        binary_scalar(DIV, out, nullptr, (float)axis, true, out, rows, s);
      }
      pool_free(partial, bucket);
      return;
    }
    const bool vec = (axis % 4) == 0;
    unsigned grid = (unsigned)((rows + 3) / 4);
    if (vec) k_row_wave<OP, true><<<grid, 256, 0, s>>>(x, mean, out, rows, (uint32_t)axis, (uint32_t)axis, true);
    else k_row_wave<OP, false><<<grid, 256, 0, s>>>(x, mean, out, rows, (uint32_t)axis, (uint32_t)axis, true);
    MALUS_HIP(hipGetLastError());
    return;
  }
  // column reduction
  const uint32_t col_blocks = (uint32_t)((inner + 255) / 256);
  size_t base_blocks = outer * col_blocks;
  uint32_t nsplit = 1;
  if (base_blocks < 1024 && axis >= 64) {
    nsplit = (uint32_t)((1024 + base_blocks - 1) / base_blocks);
    if (nsplit > axis / 16) nsplit = (uint32_t)(axis / 16 > 0 ? axis / 16 : 1);
  }
  size_t chunk = (axis + nsplit - 1) / nsplit;
  nsplit = (uint32_t)((axis + chunk - 1) / chunk);
  if (nsplit == 1) {
    k_col<OP><<<(unsigned)(base_blocks), 256, 0, s>>>(x, mean, out, outer, axis, inner, 1, chunk, col_blocks, true);
    MALUS_HIP(hipGetLastError());
    return;
  }
  size_t bucket;
  float* partial = static_cast<float*>(pool_alloc(outer * nsplit * inner * sizeof(float), &bucket));
  k_col<OP><<<(unsigned)(base_blocks * nsplit), 256, 0, s>>>(x, mean, partial, outer, axis, inner, nsplit, chunk,
                                                              col_blocks, false);
  MALUS_HIP(hipGetLastError());
  // base_blocks < 1024 here, so outer fits gridDim.y
  dim3 cgrid((unsigned)((inner + kCombCols - 1) / kCombCols), (unsigned)outer);
  k_col_combine<OP><<<cgrid, 256, 0, s>>>(partial, out, nsplit, inner, (uint32_t)axis);
  MALUS_HIP(hipGetLastError());
  pool_free(partial, bucket);
}

}  // namespace

// k_col_combine<R_VAR>/<R_MEAN> sum partials then divide: rcomb is "+" for
// both, and the element transform is applied only in the first stage.

void reduce_axis(int op, const float* x, float* out, size_t outer, size_t axis, size_t inner, hipStream_t s) {
  switch (op) {
    case R_SUM: reduce_impl<R_SUM>(x, nullptr, out, outer, axis, inner, s); break;
    case R_MEAN: reduce_impl<R_MEAN>(x, nullptr, out, outer, axis, inner, s); break;
    case R_MAX: reduce_impl<R_MAX>(x, nullptr, out, outer, axis, inner, s); break;
    case R_VAR: {
      // two-pass population variance (reduce_var.ml:11-22)
      size_t bucket;
      float* mean = static_cast<float*>(pool_alloc(outer * inner * sizeof(float), &bucket));
      reduce_impl<R_MEAN>(x, nullptr, mean, outer, axis, inner, s);
      reduce_impl<R_VAR>(x, mean, out, outer, axis, inner, s);
      pool_free(mean, bucket);
      break;
    }
    default: fail("malus: bad reduction op %d", op);
  }
}

void expand_axis(const float* small, float* out, size_t outer, size_t axis, size_t inner, hipStream_t s) {
  size_t n = outer * axis * inner;
  if (!n) return;
  size_t blocks = (n + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  k_expand_axis<<<(unsigned)blocks, 256, 0, s>>>(small, out, n, axis, inner);
  MALUS_HIP(hipGetLastError());
}

}  // namespace k
}  // namespace malus
