// Axis reductions (sum / mean / max / population variance, and the sum of a
// product) over any axis length — the reference's single-threadgroup
// kernels cap the axis at 1024 (reduce_sum.ml:13); these do not.  A
// contiguous tensor is viewed as [outer, axis, inner]:
//   inner == 1 : row reduction, one wave64 per row (shuffle tree), or a
//                two-stage split when rows are long and few;
//   inner  > 1 : column reduction.  Each workgroup owns a strip of columns
//                (float4 per thread when inner % 4 == 0) and a chunk of the
//                axis; its row-threads sum strided rows, fold through LDS in
//                fixed order, and chunk partials are combined in chunk
//                order by a second kernel.
// R_PROD sums x * y elementwise (y has x's shape): the VJP of a broadcast
// multiply reduces dout * a without materializing the product; each product
// is rounded to f32 exactly as the materialized tensor would be.
// Every order is fixed, so results are run-to-run deterministic.
#include <type_traits>
#include <utility>
#include <vector>

#include "common.h"

namespace malus {
namespace k {
namespace {

constexpr int kWave = 64;
constexpr int R_PROD = 4;
typedef float v4f __attribute__((ext_vector_type(4)));

// 128-bit loads; non-temporal when the operands exceed the 256 MB
// last-level cache (a streamed reduction input is read once), cached
// otherwise (the training step's operands are re-read by later kernels).
__device__ __forceinline__ float4 ld(const float4* p, bool nt) {
  if (nt) {
    const v4f v = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
  }
  return *p;
}
constexpr size_t kStreamBytes = 256ull << 20;

template <int OP>
__device__ __forceinline__ float rinit() { return OP == R_MAX ? -INFINITY : 0.0f; }

template <int OP>
__device__ __forceinline__ float rcomb(float a, float b) { return OP == R_MAX ? fmaxf(a, b) : a + b; }

// Element transform: VAR accumulates (x - mean)^2, PROD x * y, the rest x.
template <int OP>
__device__ __forceinline__ float rload(float x, float y, float mean) {
  if constexpr (OP == R_VAR) { float d = x - mean; return d * d; }
  else if constexpr (OP == R_PROD) return x * y;
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
// only) holds one value per row; `y` (PROD only) has x's layout.
template <int OP, bool VEC>
__global__ __launch_bounds__(256) void k_row_wave(const float* __restrict__ x, const float* __restrict__ y,
                                                  const float* __restrict__ mean, float* __restrict__ out, size_t rows,
                                                  uint32_t axis, uint32_t count, bool finalize, bool nt) {
  const size_t row = (size_t)blockIdx.x * (blockDim.x / kWave) + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (row >= rows) return;
  const float* xr = x + row * axis;
  const float* yr = OP == R_PROD ? y + row * axis : nullptr;
  const float mu = (OP == R_VAR) ? mean[row] : 0.0f;
  float acc = rinit<OP>();
  if (VEC) {
    const float4* x4 = reinterpret_cast<const float4*>(xr);
    const float4* y4 = reinterpret_cast<const float4*>(yr);
    const uint32_t n4 = axis / 4;
    for (uint32_t i = lane; i < n4; i += kWave) {
      const float4 v = ld(x4 + i, nt);
      const float4 w = OP == R_PROD ? ld(y4 + i, nt) : v;
      acc = rcomb<OP>(acc, rload<OP>(v.x, w.x, mu));
      acc = rcomb<OP>(acc, rload<OP>(v.y, w.y, mu));
      acc = rcomb<OP>(acc, rload<OP>(v.z, w.z, mu));
      acc = rcomb<OP>(acc, rload<OP>(v.w, w.w, mu));
    }
  } else {
    for (uint32_t i = lane; i < axis; i += kWave) acc = rcomb<OP>(acc, rload<OP>(xr[i], OP == R_PROD ? yr[i] : 0.f, mu));
  }
  acc = wave_reduce<OP>(acc);
  if (lane == 0) out[row] = finalize ? rfinal<OP>(acc, count) : acc;
}

// Split long rows: block (row, split) reduces [split*chunk, ...) of the row
// into partial[row * nsplit + split].
template <int OP>
__global__ __launch_bounds__(256) void k_row_split(const float* __restrict__ x, const float* __restrict__ y,
                                                   const float* __restrict__ mean, float* __restrict__ partial,
                                                   size_t axis, uint32_t nsplit, size_t chunk, bool nt) {
  __shared__ float red[256 / kWave];
  const size_t bid = blockIdx.x;
  const size_t row = bid / nsplit;
  const uint32_t sp = (uint32_t)(bid % nsplit);
  const float* xr = x + row * axis;
  const float* yr = OP == R_PROD ? y + row * axis : nullptr;
  const float mu = (OP == R_VAR) ? mean[row] : 0.0f;
  size_t beg = sp * chunk, end = beg + chunk < axis ? beg + chunk : axis;
  float acc = rinit<OP>();
  // chunk is a multiple of 4 and rows are 16-byte aligned when axis % 4 == 0
  if ((axis & 3) == 0) {
    const float4* x4 = reinterpret_cast<const float4*>(xr);
    const float4* y4 = reinterpret_cast<const float4*>(yr);
    for (size_t i = beg / 4 + threadIdx.x; i < end / 4; i += blockDim.x) {
      const float4 v = ld(x4 + i, nt);
      const float4 w = OP == R_PROD ? ld(y4 + i, nt) : v;
      acc = rcomb<OP>(acc, rload<OP>(v.x, w.x, mu));
      acc = rcomb<OP>(acc, rload<OP>(v.y, w.y, mu));
      acc = rcomb<OP>(acc, rload<OP>(v.z, w.z, mu));
      acc = rcomb<OP>(acc, rload<OP>(v.w, w.w, mu));
    }
  } else {
    for (size_t i = beg + threadIdx.x; i < end; i += blockDim.x)
      acc = rcomb<OP>(acc, rload<OP>(xr[i], OP == R_PROD ? yr[i] : 0.f, mu));
  }
  acc = wave_reduce<OP>(acc);
  if (threadIdx.x % kWave == 0) red[threadIdx.x / kWave] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float r = red[0];
    for (int w = 1; w < (int)(blockDim.x / kWave); ++w) r = rcomb<OP>(r, red[w]);
    partial[row * nsplit + sp] = r;
  }
}

// Column reduction, float4 path (inner % 4 == 0).  Block (cb, sp, o): CT
// column-threads x RT row-threads (CT * RT = 256); thread (ct, rt) owns
// columns 4 * (cb * CT + ct) .. +3 of the axis chunk [beg, end) and, in it,
// rows beg + rt, beg + rt + RT, ... (interleaved) or, with `contig`, the
// rt-th of RT contiguous runs of ceil(len / RT) rows.  Contiguous runs keep
// each wave on its own stretch of rows: on wide rows (8192 columns) the
// interleaved walk puts a block's 16 loads in flight at one column offset
// of 16 neighbouring rows, and measured 18 % slower.  The RT partial sums
// of a column are folded in rt order through LDS.  nsplit == 1 writes the
// finalized value; otherwise partial[(o * inner + i) * nsplit + sp], so
// that a column's partials form one contiguous row for the combining row
// reduction (row-major partials with k_col_combine_tree measured 3-6 %
// slower on [65536, 1024]).
template <int OP, int CT>
__global__ __launch_bounds__(256) void k_col4(const float* __restrict__ x, const float* __restrict__ y,
                                              const float* __restrict__ mean, float* __restrict__ dst, size_t axis,
                                              size_t inner, uint32_t nsplit, size_t chunk, bool finalize, bool nt,
                                              bool contig) {
  constexpr int RT = 256 / CT;
  __shared__ float4 red[RT][CT];
  const int ct = threadIdx.x % CT, rt = threadIdx.x / CT;
  const uint32_t sp = blockIdx.y;
  const size_t o = blockIdx.z;
  const size_t i4 = (size_t)blockIdx.x * CT + ct;  // float4 column group
  const bool live = 4 * i4 < inner;
  float4 acc = make_float4(rinit<OP>(), rinit<OP>(), rinit<OP>(), rinit<OP>());
  if (live) {
    float4 mu = make_float4(0.f, 0.f, 0.f, 0.f);
    if (OP == R_VAR) mu = reinterpret_cast<const float4*>(mean + o * inner)[i4];
    const size_t beg = sp * chunk, end = beg + chunk < axis ? beg + chunk : axis;
    const float4* xp = reinterpret_cast<const float4*>(x + o * axis * inner) + i4;
    const float4* yp = OP == R_PROD ? reinterpret_cast<const float4*>(y + o * axis * inner) + i4 : nullptr;
    const size_t stride4 = inner / 4;
    auto fold = [&](float4 v, float4 w) {
      acc.x = rcomb<OP>(acc.x, rload<OP>(v.x, w.x, mu.x));
      acc.y = rcomb<OP>(acc.y, rload<OP>(v.y, w.y, mu.y));
      acc.z = rcomb<OP>(acc.z, rload<OP>(v.z, w.z, mu.z));
      acc.w = rcomb<OP>(acc.w, rload<OP>(v.w, w.w, mu.w));
    };
    size_t a = beg + rt, aend = end, step = RT;
    if (contig) {
      const size_t run = (end - beg + RT - 1) / RT;
      a = beg + rt * run;
      aend = a + run < end ? a + run : end;
      step = 1;
    }
    // four rows' loads in flight before their (in-order) folds
    for (; a + 3 * step < aend; a += 4 * step) {
      float4 v[4], w[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        v[u] = ld(xp + (a + u * step) * stride4, nt);
        w[u] = OP == R_PROD ? ld(yp + (a + u * step) * stride4, nt) : v[u];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) fold(v[u], w[u]);
    }
    for (; a < aend; a += step) {
      const float4 v = ld(xp + a * stride4, nt);
      fold(v, OP == R_PROD ? ld(yp + a * stride4, nt) : v);
    }
  }
  red[rt][ct] = acc;
  __syncthreads();
  if (rt == 0 && live) {
    float4 r = red[0][ct];
#pragma unroll
    for (int k = 1; k < RT; ++k) {
      const float4 q = red[k][ct];
      r.x = rcomb<OP>(r.x, q.x);
      r.y = rcomb<OP>(r.y, q.y);
      r.z = rcomb<OP>(r.z, q.z);
      r.w = rcomb<OP>(r.w, q.w);
    }
    if (nsplit == 1) {
      if (finalize) {
        r.x = rfinal<OP>(r.x, (uint32_t)axis);
        r.y = rfinal<OP>(r.y, (uint32_t)axis);
        r.z = rfinal<OP>(r.z, (uint32_t)axis);
        r.w = rfinal<OP>(r.w, (uint32_t)axis);
      }
      reinterpret_cast<float4*>(dst + o * inner)[i4] = r;
    } else {  // split partials column-major: column c's nsplit partials are contiguous
      float* pc = dst + (o * inner + 4 * i4) * nsplit + sp;
      pc[0] = r.x;
      pc[nsplit] = r.y;
      pc[2 * (size_t)nsplit] = r.z;
      pc[3 * (size_t)nsplit] = r.w;
    }
  }
}

// Column reduction, scalar path: thread handles one column i for the axis
// chunk [sp*chunk, ...).
template <int OP>
__global__ __launch_bounds__(256) void k_col(const float* __restrict__ x, const float* __restrict__ y,
                                             const float* __restrict__ mean, float* __restrict__ dst, size_t outer,
                                             size_t axis, size_t inner, uint32_t nsplit, size_t chunk,
                                             uint32_t col_blocks, bool finalize) {
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
  const float* yp = OP == R_PROD ? y + o * axis * inner + i : nullptr;
  float acc = rinit<OP>();
  for (size_t a = beg; a < end; ++a) acc = rcomb<OP>(acc, rload<OP>(xp[a * inner], OP == R_PROD ? yp[a * inner] : 0.f, mu));
  if (nsplit == 1) dst[o * inner + i] = finalize ? rfinal<OP>(acc, (uint32_t)axis) : acc;
  else dst[(o * nsplit + sp) * inner + i] = acc;
}

// Combine the split partials of a column reduction: CC columns per block,
// G = 256 / CC split groups each summing every G-th partial in split order
// (four loads in flight), then a fixed pairwise tree over the groups.  CC is
// picked so that every group sums a few partials; the order depends only on
// the shape, so the result is deterministic.
template <int OP, int CC>
__global__ __launch_bounds__(256) void k_col_combine(const float* __restrict__ partial, float* __restrict__ out,
                                                     uint32_t nsplit, size_t inner, uint32_t count) {
  constexpr int G = 256 / CC;
  __shared__ float red[G][CC];
  const int lc = threadIdx.x % CC, g = threadIdx.x / CC;
  const size_t o = blockIdx.y;
  const size_t i = (size_t)blockIdx.x * CC + lc;
  float acc = rinit<OP>();
  if (i < inner) {
    const float* p = partial + o * nsplit * inner + i;
    uint32_t sp = g;
    for (; sp + 3 * G < nsplit; sp += 4 * G) {
      float v[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) v[u] = p[(size_t)(sp + u * G) * inner];
#pragma unroll
      for (int u = 0; u < 4; ++u) acc = rcomb<OP>(acc, v[u]);
    }
    for (; sp < nsplit; sp += G) acc = rcomb<OP>(acc, p[(size_t)sp * inner]);
  }
  red[g][lc] = acc;
  __syncthreads();
#pragma unroll
  for (int w = G / 2; w > 0; w >>= 1) {
    if (g < w) red[g][lc] = rcomb<OP>(red[g][lc], red[g + w][lc]);
    __syncthreads();
  }
  if (g == 0 && i < inner) out[o * inner + i] = rfinal<OP>(red[0][lc], count);
}

// Combine split partials stored row-major ([o][sp][inner]: the layernorm
// VJP's column partials, one contiguous row per split) in the order
// k_row_wave<OP, VEC> reduces the same values stored column-major (a
// column's nsplit partials contiguous, as k_col4 writes them): lane slot l
// (0..63) folds, from rinit, the partials l, l + 64, ... (VEC: the runs of
// four 4l .. 4l + 3, 4 (l + 64) .., one float4 per lane step) in order, then
// the 64 slot sums go through wave_reduce's butterfly as lane 0 sees it
// (level w: slot l += slot l + w for l < w, w = 32 .. 1).  So both layouts
// give the same sums, bit for bit.  CC columns per block, G = 256 / CC slot
// groups, 64 / G slots per thread.
// col_combine_tree_cols: columns [bx CC, bx CC + CC) of one [nsplit][inner]
// partial block into out[0 .. inner).
template <int OP, bool VEC, int CC>
__device__ __forceinline__ void col_combine_tree_cols(const float* __restrict__ partial, float* __restrict__ out,
                                                      uint32_t nsplit, size_t inner, uint32_t count, size_t bx) {
  constexpr int G = 256 / CC, LPT = kWave / G;
  static_assert(kWave % G == 0, "whole lane slots per thread");
  __shared__ float red[kWave][CC];
  const int lc = threadIdx.x % CC, g = threadIdx.x / CC;
  const size_t i = bx * CC + lc;
  const float* p = partial + i;
  // step k reads, for every slot of the thread, its k-th run (VEC: four
  // partials, else one) before folding any of them: one memory round trip
  // per step
  constexpr int RUN = VEC ? 4 : 1;
  const uint32_t runs = VEC ? nsplit / 4 : nsplit;
  float acc[LPT];
#pragma unroll
  for (int u = 0; u < LPT; ++u) acc[u] = rinit<OP>();
  if (i < inner) {
    for (uint32_t q0 = 0; q0 < runs; q0 += kWave) {
      float v[LPT][RUN];
#pragma unroll
      for (int u = 0; u < LPT; ++u) {
        const uint32_t q = q0 + g + u * G;
#pragma unroll
        for (int e = 0; e < RUN; ++e) v[u][e] = q < runs ? p[(size_t)(RUN * q + e) * inner] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < LPT; ++u) {
        if (q0 + g + u * G < runs) {
#pragma unroll
          for (int e = 0; e < RUN; ++e) acc[u] = rcomb<OP>(acc[u], v[u][e]);
        }
      }
    }
  }
#pragma unroll
  for (int u = 0; u < LPT; ++u) red[g + u * G][lc] = acc[u];
  __syncthreads();
#pragma unroll
  for (int w = kWave / 2; w > 0; w >>= 1) {
#pragma unroll
    for (int u = 0; u < LPT; ++u) {
      const int l = g + u * G;
      if (l < w) red[l][lc] = rcomb<OP>(red[l][lc], red[l + w][lc]);
    }
    __syncthreads();
  }
  if (g == 0 && i < inner) out[i] = rfinal<OP>(red[0][lc], count);
}

template <int OP, bool VEC, int CC>
__global__ __launch_bounds__(256) void k_col_combine_tree(const float* __restrict__ partial, float* __restrict__ out,
                                                          uint32_t nsplit, size_t inner, uint32_t count) {
  const size_t o = blockIdx.y;
  col_combine_tree_cols<OP, VEC, CC>(partial + o * nsplit * inner, out + o * inner, nsplit, inner, count, blockIdx.x);
}

// Several column sums (nsplit % 4 == 0) in one launch: block (x, j) runs
// column block x of job j, the same sums k_col_combine_tree forms for it
// alone.
struct ColSumJobs {
  static constexpr int kMax = 32;
  const float* partial[kMax];
  float* out[kMax];
  uint32_t nsplit[kMax], inner[kMax], count[kMax];
};

template <int CC>
__global__ __launch_bounds__(256) void k_col_combine_tree_jobs(const ColSumJobs jobs) {
  const int j = blockIdx.y;
  if ((size_t)blockIdx.x * CC >= jobs.inner[j]) return;  // the grid spans the widest job
  col_combine_tree_cols<R_SUM, true, CC>(jobs.partial[j], jobs.out[j], jobs.nsplit[j], jobs.inner[j], jobs.count[j],
                                         blockIdx.x);
}

// Launch k_col_combine_tree over [outer][nsplit][inner] partials.
template <int OP>
void launch_col_combine_tree(const float* partial, float* out, size_t outer, uint32_t nsplit, size_t inner,
                             uint32_t count, hipStream_t s) {
  constexpr int CC = 8;  // 4.4 us for the C5 layernorm scale (384 columns, 512 splits); 16: 5.5 us
  const dim3 grid((unsigned)((inner + CC - 1) / CC), (unsigned)outer);
  if (nsplit % 4 == 0) k_col_combine_tree<OP, true, CC><<<grid, 256, 0, s>>>(partial, out, nsplit, inner, count);
  else k_col_combine_tree<OP, false, CC><<<grid, 256, 0, s>>>(partial, out, nsplit, inner, count);
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

// The partials of MEAN / VAR / PROD are plain sums: combine them with SUM
// (finalizing divides where the op needs it).
template <int OP>
constexpr int combine_op() { return OP == R_MAX ? R_MAX : OP == R_PROD ? R_SUM : OP; }

template <int OP>
void launch_col4(int ct, dim3 grid, const float* x, const float* y, const float* mean, float* dst, size_t axis,
                 size_t inner, uint32_t nsplit, size_t chunk, bool finalize, bool nt, bool contig, hipStream_t s) {
  switch (ct) {
    case 8: k_col4<OP, 8><<<grid, 256, 0, s>>>(x, y, mean, dst, axis, inner, nsplit, chunk, finalize, nt, contig); break;
    case 16: k_col4<OP, 16><<<grid, 256, 0, s>>>(x, y, mean, dst, axis, inner, nsplit, chunk, finalize, nt, contig); break;
    case 32: k_col4<OP, 32><<<grid, 256, 0, s>>>(x, y, mean, dst, axis, inner, nsplit, chunk, finalize, nt, contig); break;
    default: k_col4<OP, 64><<<grid, 256, 0, s>>>(x, y, mean, dst, axis, inner, nsplit, chunk, finalize, nt, contig); break;
  }
}

// The column reduction's launch plan for [outer, axis, inner] (inner > 1):
// float4 path (vec) with CT column-threads x 256/CT row-threads per block, or
// the scalar path; the axis split into nsplit chunks of `chunk` rows until
// the grid holds ~2048 workgroups, keeping >= 4 rows per row-thread (vec) or
// >= 16 rows per thread (scalar).  Row-threads walk contiguous runs once a
// run holds >= 16 rows (contig); shorter chunks keep the interleaved walk.
// CT = 32 (512-byte row segments, 8 row-threads) measured fastest with the
// contiguous runs on [8192, 8192] and [65536, 1024] (6.1 and 6.5 TB/s for
// the partial pass).
struct ColPlan {
  bool vec;
  int ct;
  size_t col_blocks;
  uint32_t nsplit;
  size_t chunk;
  bool contig;
};
ColPlan col_plan(size_t outer, size_t axis, size_t inner, bool aligned) {
  ColPlan p{};
  p.vec = inner % 4 == 0 && outer <= 65535 && aligned;
  p.ct = 32;
  if (p.vec) {
    const size_t groups = inner / 4;  // float4 columns
    while (p.ct > 8 && groups % p.ct != 0) p.ct >>= 1;
    if (groups % p.ct != 0) p.ct = 32;
    p.col_blocks = (groups + p.ct - 1) / p.ct;
  } else {
    p.col_blocks = (inner + 255) / 256;
  }
  const size_t base_blocks = outer * p.col_blocks;
  const size_t rows_per_block = p.vec ? (size_t)(256 / p.ct) * 4 : 16;
  p.nsplit = 1;
  if (base_blocks < 2048) {
    size_t want = (2048 + base_blocks - 1) / base_blocks;
    size_t cap = axis / rows_per_block > 0 ? axis / rows_per_block : 1;
    p.nsplit = (uint32_t)(want < cap ? want : cap);
    if (p.nsplit > 65535) p.nsplit = 65535;
  }
  p.chunk = (axis + p.nsplit - 1) / p.nsplit;
  p.nsplit = (uint32_t)((axis + p.chunk - 1) / p.chunk);
  p.contig = p.vec && p.chunk >= (size_t)16 * (256 / p.ct);
  return p;
}

// Where a reduction's temporaries (split partials, the variance's mean) come
// from: the device pool by default, or a caller's fixed buffer (`base`, `cap`
// floats), carved in 256-byte-aligned pieces.  Buffers taken from the pool
// go back to it in release(): stream order keeps every later user behind the
// kernels that read them.
struct Arena {
  float* base = nullptr;
  size_t cap = 0, used = 0;
  std::vector<std::pair<void*, size_t>> pooled;
  float* get(size_t n) {
    if (!base) {
      size_t bucket;
      void* p = pool_alloc(n * sizeof(float), &bucket);
      pooled.emplace_back(p, bucket);
      return static_cast<float*>(p);
    }
    if (used + n > cap) fail("malus: reduction scratch overflow (%zu + %zu floats > %zu)", used, n, cap);
    float* p = base + used;
    used += (n + 63) / 64 * 64;
    return p;
  }
  void release() {
    for (auto& q : pooled) pool_free(q.first, q.second);
    pooled.clear();
  }
};

// The split plan of a long-row reduction (rows of `axis` elements): 0 when
// the rows are reduced without splitting.
uint32_t row_split(size_t rows, size_t axis, size_t* chunk_out) {
  if (!(axis >= 16384 && rows < 2048)) return 0;
  size_t want_blocks = 2048;
  uint32_t nsplit = (uint32_t)((want_blocks + rows - 1) / rows);
  size_t chunk = (axis + nsplit - 1) / nsplit;
  chunk = (chunk + 1023) / 1024 * 1024;  // multiple of 4, float4-friendly
  nsplit = (uint32_t)((axis + chunk - 1) / chunk);
  *chunk_out = chunk;
  return nsplit;
}

// Floats of partials one reduce_impl call takes from its arena.
size_t partial_floats(size_t outer, size_t axis, size_t inner, bool aligned) {
  if (outer * inner == 0 || axis == 0) return 0;
  if (inner == 1) {
    size_t chunk;
    const uint32_t nsplit = row_split(outer, axis, &chunk);
    return nsplit ? outer * nsplit : 0;
  }
  const ColPlan cp = col_plan(outer, axis, inner, aligned);
  return cp.nsplit > 1 ? (outer * cp.nsplit * inner + 63) / 64 * 64 : 0;
}

template <int OP>
void reduce_impl(const float* x, const float* y, const float* mean, float* out, size_t outer, size_t axis, size_t inner,
                 hipStream_t s, Arena& arena) {
  constexpr int COMB = combine_op<OP>();
  const size_t n_out = outer * inner;
  const bool nt = outer * axis * inner * sizeof(float) * (OP == R_PROD ? 2 : 1) >= kStreamBytes;
  if (n_out == 0) return;
  if (axis == 0) {  // empty reduction: sum/mean identities (mean/var of nothing -> NaN like 0/0)
    if (OP == R_MAX) fill(out, -INFINITY, n_out, s);
    else if (OP == R_SUM || OP == R_PROD) fill(out, 0.0f, n_out, s);
    else fill(out, NAN, n_out, s);
    return;
  }
  if (inner == 1) {
    const size_t rows = outer;
    // Long rows with few of them: split each row across blocks.
    size_t chunk;
    if (const uint32_t nsplit = row_split(rows, axis, &chunk)) {
      float* partial = arena.get(rows * nsplit);
      k_row_split<OP><<<(unsigned)(rows * nsplit), 256, 0, s>>>(x, y, mean, partial, axis, nsplit, chunk, nt);
      MALUS_HIP(hipGetLastError());
      // combine partials of each row with one wave per row; MEAN and VAR
      // divide the combined sum by the axis length in the same kernel
      constexpr int FIN = COMB == R_MAX ? R_MAX : (OP == R_MEAN || OP == R_VAR) ? R_MEAN : R_SUM;
      k_row_wave<FIN, false><<<(unsigned)((rows + 3) / 4), 256, 0, s>>>(partial, nullptr, nullptr, out, rows, nsplit,
                                                                       (uint32_t)axis, true, false);
      MALUS_HIP(hipGetLastError());
      return;
    }
    const bool vec = (axis % 4) == 0;
    unsigned grid = (unsigned)((rows + 3) / 4);
    if (vec) k_row_wave<OP, true><<<grid, 256, 0, s>>>(x, y, mean, out, rows, (uint32_t)axis, (uint32_t)axis, true, nt);
    else k_row_wave<OP, false><<<grid, 256, 0, s>>>(x, y, mean, out, rows, (uint32_t)axis, (uint32_t)axis, true, nt);
    MALUS_HIP(hipGetLastError());
    return;
  }
  // column reduction
  const bool aligned = ((uintptr_t)x | (uintptr_t)y | (uintptr_t)mean | (uintptr_t)out) % 16 == 0;
  const ColPlan cp = col_plan(outer, axis, inner, aligned);
  const bool vec = cp.vec;
  const int ct = cp.ct;
  const size_t col_blocks = cp.col_blocks, base_blocks = outer * col_blocks, chunk = cp.chunk;
  const uint32_t nsplit = cp.nsplit;
  float* dst = out;
  if (nsplit > 1) dst = arena.get(outer * nsplit * inner);
  if (vec) {
    launch_col4<OP>(ct, dim3((unsigned)col_blocks, nsplit, (unsigned)outer), x, y, mean, dst, axis, inner, nsplit, chunk,
                    nsplit == 1, nt, cp.contig, s);
  } else {
    k_col<OP><<<(unsigned)(base_blocks * nsplit), 256, 0, s>>>(x, y, mean, dst, outer, axis, inner, nsplit, chunk,
                                                                (uint32_t)col_blocks, nsplit == 1);
  }
  MALUS_HIP(hipGetLastError());
  if (nsplit > 1 && vec) {
    // one wave per column over its contiguous partials (MEAN and VAR divide
    // the combined sum by the axis length in the same kernel)
    constexpr int FIN = COMB == R_MAX ? R_MAX : (OP == R_MEAN || OP == R_VAR) ? R_MEAN : R_SUM;
    const size_t cols = outer * inner;
    if (nsplit % 4 == 0)
      k_row_wave<FIN, true><<<(unsigned)((cols + 3) / 4), 256, 0, s>>>(dst, nullptr, nullptr, out, cols, nsplit,
                                                                        (uint32_t)axis, true, false);
    else
      k_row_wave<FIN, false><<<(unsigned)((cols + 3) / 4), 256, 0, s>>>(dst, nullptr, nullptr, out, cols, nsplit,
                                                                         (uint32_t)axis, true, false);
    MALUS_HIP(hipGetLastError());
  } else if (nsplit > 1) {
    // base_blocks < 2048 here, so outer fits gridDim.y
    // columns per combine block: enough split groups to keep ~4+ partials each
    const int cc = nsplit >= 256 ? 4 : nsplit >= 64 ? 16 : 64;
    dim3 cgrid((unsigned)((inner + cc - 1) / cc), (unsigned)outer);
    auto comb = [&](auto tag) {
      constexpr int C = decltype(tag)::value;
      const uint32_t cnt = (uint32_t)axis;
      if (OP == R_MAX) k_col_combine<R_MAX, C><<<cgrid, 256, 0, s>>>(dst, out, nsplit, inner, cnt);
      else if (OP == R_MEAN || OP == R_VAR) k_col_combine<R_MEAN, C><<<cgrid, 256, 0, s>>>(dst, out, nsplit, inner, cnt);
      else k_col_combine<R_SUM, C><<<cgrid, 256, 0, s>>>(dst, out, nsplit, inner, cnt);
    };
    if (cc == 4) comb(std::integral_constant<int, 4>{});
    else if (cc == 16) comb(std::integral_constant<int, 16>{});
    else comb(std::integral_constant<int, 64>{});
    MALUS_HIP(hipGetLastError());
  }
}

}  // namespace

static void reduce_axis_in(int op, const float* x, float* out, size_t outer, size_t axis, size_t inner, hipStream_t s,
                           Arena& arena) {
  switch (op) {
    case R_SUM: reduce_impl<R_SUM>(x, nullptr, nullptr, out, outer, axis, inner, s, arena); break;
    case R_MEAN: reduce_impl<R_MEAN>(x, nullptr, nullptr, out, outer, axis, inner, s, arena); break;
    case R_MAX: reduce_impl<R_MAX>(x, nullptr, nullptr, out, outer, axis, inner, s, arena); break;
    case R_VAR: {
      // two-pass population variance (reduce_var.ml:11-22); the mean pass's
      // partials are consumed before the variance pass starts (stream order),
      // so both passes carve the same region after the mean
      float* mean = arena.get(outer * inner);
      const size_t mark = arena.used;
      reduce_impl<R_MEAN>(x, nullptr, nullptr, mean, outer, axis, inner, s, arena);
      arena.used = mark;
      reduce_impl<R_VAR>(x, nullptr, mean, out, outer, axis, inner, s, arena);
      break;
    }
    default: fail("malus: bad reduction op %d", op);
  }
}

void reduce_axis(int op, const float* x, float* out, size_t outer, size_t axis, size_t inner, hipStream_t s) {
  Arena arena;
  reduce_axis_in(op, x, out, outer, axis, inner, s, arena);
  arena.release();
}

size_t reduce_axis_scratch_floats(int op, const float* x, const float* out, size_t outer, size_t axis, size_t inner) {
  // each pass plans with the pointers it is given (reduce_impl): a plain
  // reduction with x and out; the variance's mean pass with x and the
  // 256-byte-aligned mean, its second pass with x, the mean and out
  const bool aligned = ((uintptr_t)x | (uintptr_t)out) % 16 == 0;
  const size_t part = partial_floats(outer, axis, inner, aligned);
  if (op != R_VAR) return part;
  const size_t mean_part = partial_floats(outer, axis, inner, (uintptr_t)x % 16 == 0);
  return (outer * inner + 63) / 64 * 64 + (part > mean_part ? part : mean_part);
}

void reduce_axis_scratch(int op, const float* x, float* out, size_t outer, size_t axis, size_t inner, float* scratch,
                         size_t scratch_floats, hipStream_t s) {
  Arena arena;
  arena.base = scratch;
  arena.cap = scratch_floats;
  reduce_axis_in(op, x, out, outer, axis, inner, s, arena);
}

void reduce_axis_prod(const float* x, const float* y, float* out, size_t outer, size_t axis, size_t inner, hipStream_t s) {
  Arena arena;
  reduce_impl<R_PROD>(x, y, nullptr, out, outer, axis, inner, s, arena);
  arena.release();
}

bool col_prod_split(size_t axis, size_t inner, uint32_t* nsplit, size_t* chunk, int* row_threads) {
  if (inner <= 1) return false;
  const ColPlan p = col_plan(1, axis, inner, true);
  if (!p.vec || p.nsplit < 2 || p.contig) return false;  // the interleaved walk only
  *nsplit = p.nsplit;
  *chunk = p.chunk;
  *row_threads = 256 / p.ct;
  return true;
}

void col_combine_sum(const float* partial, float* out, size_t cols, uint32_t nsplit, size_t axis, hipStream_t s) {
  launch_col_combine_tree<R_SUM>(partial, out, 1, nsplit, cols, (uint32_t)axis, s);
  MALUS_HIP(hipGetLastError());
}

namespace {
struct DeferredColSum {
  float* partial;
  size_t bucket;
  float* out;
  uint32_t nsplit, inner, count;
};
thread_local std::vector<DeferredColSum> t_colsums;
}  // namespace

void col_combine_sum_owned(float* partial, size_t bucket, float* out, size_t cols, uint32_t nsplit, size_t axis,
                           bool defer, hipStream_t s) {
  if (defer && nsplit % 4 == 0 && cols <= UINT32_MAX && axis <= UINT32_MAX) {
    t_colsums.push_back({partial, bucket, out, nsplit, (uint32_t)cols, (uint32_t)axis});
    return;
  }
  col_combine_sum(partial, out, cols, nsplit, axis, s);
  pool_free(partial, bucket);
}

void col_combine_flush(hipStream_t s) {
  std::vector<DeferredColSum> jobs;
  jobs.swap(t_colsums);
  constexpr int CC = 8;  // as launch_col_combine_tree
  try {
    for (size_t b = 0; b < jobs.size(); b += ColSumJobs::kMax) {
      const int n = (int)std::min<size_t>(ColSumJobs::kMax, jobs.size() - b);
      ColSumJobs t{};
      uint32_t widest = 0;
      for (int j = 0; j < n; ++j) {
        const DeferredColSum& d = jobs[b + j];
        t.partial[j] = d.partial;
        t.out[j] = d.out;
        t.nsplit[j] = d.nsplit;
        t.inner[j] = d.inner;
        t.count[j] = d.count;
        widest = std::max(widest, d.inner);
      }
      k_col_combine_tree_jobs<CC><<<dim3((widest + CC - 1) / CC, (unsigned)n), 256, 0, s>>>(t);
      MALUS_HIP(hipGetLastError());
    }
  } catch (...) {
    for (const DeferredColSum& d : jobs) pool_free(d.partial, d.bucket);
    throw;
  }
  for (const DeferredColSum& d : jobs) pool_free(d.partial, d.bucket);
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
