// Row kernels: softmax, layernorm, cross-entropy (forward and VJP).
// Contiguous rows (inner == 1) up to 4096 wide run one wave64 per row with
// the whole row held in registers: one HBM read per input element and one
// write per output element, reductions by wave shuffles.  Other shapes
// (reductions over a non-last axis, rows wider than 4096) use a sequential
// per-(outer, inner) kernel that follows the reference loops directly.
#include "common.h"

namespace malus {
namespace k {
namespace {

constexpr int kWave = 64;
constexpr int kRowsPerBlock = 4;  // 256 threads
typedef float v4f __attribute__((ext_vector_type(4)));  // non-temporal 128-bit row access

__device__ __forceinline__ float wsum(float v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}
__device__ __forceinline__ float wmax(float v) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

// Register tile of one row: NV float4 chunks per lane.  Element e of the
// lane's tile is column col(e).  VM: 0 scalar, 1 float4, 2 float4 with
// non-temporal loads (for operands too large to stay in the 256 MB
// last-level cache between kernels).  VEC: chunk j covers columns 4*(lane+64j)..+3;
// scalar: element e is column lane + 64*e.
template <int NV, int VM>
struct RowTile {
  static constexpr bool VEC = VM > 0, NT = VM == 2;
  float v[NV * 4];
  __device__ __forceinline__ static uint32_t col(int e, int lane) {
    return VEC ? 4u * (uint32_t)(lane + kWave * (e / 4)) + (uint32_t)(e % 4) : (uint32_t)(lane + kWave * e);
  }
  __device__ __forceinline__ void load(const float* __restrict__ row, uint32_t axis, int lane, float pad) {
    if (VEC) {
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        uint32_t c4 = (uint32_t)(lane + kWave * j);
        if (4 * c4 < axis) {
          const v4f t = NT ? __builtin_nontemporal_load(reinterpret_cast<const v4f*>(row) + c4)
                           : reinterpret_cast<const v4f*>(row)[c4];
          v[4 * j] = t.x; v[4 * j + 1] = t.y; v[4 * j + 2] = t.z; v[4 * j + 3] = t.w;
        } else {
          v[4 * j] = v[4 * j + 1] = v[4 * j + 2] = v[4 * j + 3] = pad;
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < NV * 4; ++e) {
        uint32_t c = col(e, lane);
        v[e] = c < axis ? row[c] : pad;
      }
    }
  }
  __device__ __forceinline__ void store(float* __restrict__ row, uint32_t axis, int lane) const {
    if (VEC) {
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        uint32_t c4 = (uint32_t)(lane + kWave * j);
        // ordinary store: the next op (often a GEMM) reads this row back from cache
        if (4 * c4 < axis) reinterpret_cast<float4*>(row)[c4] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < NV * 4; ++e) {
        uint32_t c = col(e, lane);
        if (c < axis) row[c] = v[e];
      }
    }
  }
  __device__ __forceinline__ bool valid(int e, int lane, uint32_t axis) const { return col(e, lane) < axis; }
};

// softmax_axis_cpu (metal.rs:1439-1467): m = max, e = exp(x - m), s = sum e, y = e / s
template <int NV, int VM>
__global__ __launch_bounds__(256) void k_softmax_rows(const float* __restrict__ x, float* __restrict__ y, size_t rows,
                                                      uint32_t axis) {
  const size_t row = (size_t)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (row >= rows) return;
  RowTile<NV, VM> t;
  t.load(x + row * axis, axis, lane, -INFINITY);
  float m = -INFINITY;
#pragma unroll
  for (int e = 0; e < NV * 4; ++e) m = fmaxf(m, t.v[e]);
  m = wmax(m);
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < NV * 4; ++e) {
    float ex = t.valid(e, lane, axis) ? expf(t.v[e] - m) : 0.0f;
    t.v[e] = ex;
    s += ex;
  }
  s = wsum(s);
#pragma unroll
  for (int e = 0; e < NV * 4; ++e) t.v[e] = t.v[e] / s;
  t.store(y + row * axis, axis, lane);
}

// Attention scores: y = softmax((x * scale[0]) + mask[row % mask_rows]) over
// the row, fusing nanogpt_modular.ml's `scores * scale`, `+ mask` and
// softmax.  Each op rounds like its own kernel (the product, then the sum,
// then softmax_axis_cpu), so y equals the three-kernel result bit for bit.
template <int NV, int VM>
__global__ __launch_bounds__(256) void k_scale_mask_softmax_rows(const float* __restrict__ x, const float* __restrict__ scale,
                                                                 const float* __restrict__ mask, float* __restrict__ y,
                                                                 size_t rows, uint32_t axis, uint32_t mask_rows) {
  const size_t row = (size_t)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (row >= rows) return;
  const float sc = scale[0];
  RowTile<NV, VM> t, mk;
  t.load(x + row * axis, axis, lane, 0.0f);
  mk.load(mask + (row % mask_rows) * axis, axis, lane, 0.0f);
#pragma unroll
  for (int e = 0; e < NV * 4; ++e) {
    const float ss = t.v[e] * sc;
    t.v[e] = t.valid(e, lane, axis) ? ss + mk.v[e] : -INFINITY;
  }
  float m = -INFINITY;
#pragma unroll
  for (int e = 0; e < NV * 4; ++e) m = fmaxf(m, t.v[e]);
  m = wmax(m);
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < NV * 4; ++e) {
    float ex = t.valid(e, lane, axis) ? expf(t.v[e] - m) : 0.0f;
    t.v[e] = ex;
    s += ex;
  }
  s = wsum(s);
#pragma unroll
  for (int e = 0; e < NV * 4; ++e) t.v[e] = t.v[e] / s;
  t.store(y + row * axis, axis, lane);
}

// tape.rs:1150-1161: dx = s * (dout - sum(dout * s))
template <int NV, int VM>
__global__ __launch_bounds__(256) void k_softmax_bwd_rows(const float* __restrict__ y, const float* __restrict__ dout,
                                                          float* __restrict__ dx, size_t rows, uint32_t axis) {
  const size_t row = (size_t)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (row >= rows) return;
  RowTile<NV, VM> s, d;
  s.load(y + row * axis, axis, lane, 0.0f);
  d.load(dout + row * axis, axis, lane, 0.0f);
  float acc = 0.0f;
#pragma unroll
  for (int e = 0; e < NV * 4; ++e) { float p = d.v[e] * s.v[e]; acc += p; }
  acc = wsum(acc);
#pragma unroll
  for (int e = 0; e < NV * 4; ++e) { float diff = d.v[e] - acc; s.v[e] = s.v[e] * diff; }
  s.store(dx + row * axis, axis, lane);
}

// tensor_layernorm_axis (metal.rs:1486-1533): y = (x - mu) / sqrt(var + eps)
// With w: also out = y * w[col] (the `layernorm(x) * w` of nanogpt_modular.ml:47,
// rounded like the separate broadcast multiply).
template <int NV, int VM>
__global__ __launch_bounds__(256) void k_layernorm_rows(const float* __restrict__ x, float* __restrict__ y,
                                                        float* __restrict__ var, size_t rows, uint32_t axis, float eps,
                                                        const float* __restrict__ w, float* __restrict__ out) {
  const size_t row = (size_t)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (row >= rows) return;
  RowTile<NV, VM> t;
  t.load(x + row * axis, axis, lane, 0.0f);
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < NV * 4; ++e) s += t.v[e];
  s = wsum(s);
  const float mu = s / (float)axis;
  float q = 0.0f;
#pragma unroll
  for (int e = 0; e < NV * 4; ++e) {
    if (t.valid(e, lane, axis)) { float dd = t.v[e] - mu; q += dd * dd; }
  }
  q = wsum(q);
  const float va = q / (float)axis;
  const float sigma = sqrtf(va + eps);
#pragma unroll
  for (int e = 0; e < NV * 4; ++e) t.v[e] = (t.v[e] - mu) / sigma;
  t.store(y + row * axis, axis, lane);
  if (lane == 0 && var) var[row] = va;
  if (w) {
    RowTile<NV, VM == 2 ? 1 : VM> wt;  // w is re-read by every row: cached loads
    wt.load(w, axis, lane, 0.0f);
#pragma unroll
    for (int e = 0; e < NV * 4; ++e) t.v[e] = t.v[e] * wt.v[e];
    t.store(out + row * axis, axis, lane);
  }
}

// tape.rs:1162-1186: dx = ((dy - mean(dy)) - y * mean(dy*y)) * (1 / sqrt(var + eps))
template <int NV, int VM>
__global__ __launch_bounds__(256) void k_layernorm_bwd_rows(const float* __restrict__ y, const float* __restrict__ var,
                                                            const float* __restrict__ dout, float* __restrict__ dx,
                                                            size_t rows, uint32_t axis, float eps,
                                                            const float* __restrict__ addend,
                                                            const float* __restrict__ w) {
  const size_t row = (size_t)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (row >= rows) return;
  RowTile<NV, VM> yt, dt;
  yt.load(y + row * axis, axis, lane, 0.0f);
  dt.load(dout + row * axis, axis, lane, 0.0f);
  if (w) {  // dout is the gradient of y * w: dy = dout * w, rounded like the multiply's VJP
    RowTile<NV, VM == 2 ? 1 : VM> wt;
    wt.load(w, axis, lane, 0.0f);
#pragma unroll
    for (int e = 0; e < NV * 4; ++e) dt.v[e] = dt.v[e] * wt.v[e];
  }
  float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
  for (int e = 0; e < NV * 4; ++e) { s1 += dt.v[e]; float p = dt.v[e] * yt.v[e]; s2 += p; }
  s1 = wsum(s1);
  s2 = wsum(s2);
  const float dy_mean = s1 / (float)axis;
  const float dyy_mean = s2 / (float)axis;
  const float inv_sigma = 1.0f / sqrtf(var[row] + eps);
#pragma unroll
  for (int e = 0; e < NV * 4; ++e) {
    float y_term = yt.v[e] * dyy_mean;
    float tmp = dt.v[e] - dy_mean;
    float numer = tmp - y_term;
    yt.v[e] = numer * inv_sigma;
  }
  if (addend) {  // gradient accumulation: old + this VJP's value
    dt.load(addend + row * axis, axis, lane, 0.0f);
#pragma unroll
    for (int e = 0; e < NV * 4; ++e) yt.v[e] = dt.v[e] + yt.v[e];
  }
  yt.store(dx + row * axis, axis, lane);
}

// Half-wave forms of the two layernorm kernels for rows of 128 * NV floats
// (NV <= 4: the C = 128 .. 512 models): 32 lanes per row, NV float4 per lane
// with no idle lanes, eight rows per workgroup.  Same arithmetic as the
// full-wave kernels above; the sums run over 32 lanes instead of 64.
__device__ __forceinline__ float hsum(float v) {
#pragma unroll
  for (int off = 16; off > 0; off >>= 1) v += __shfl_xor(v, off, 32);
  return v;
}
constexpr int kHalfRowsPerBlock = 8;

// OB: out stored in bf16 (each product rounded to nearest even).
template <int NV, bool OB = false>
__global__ __launch_bounds__(256) void k_layernorm_rows32(const float* __restrict__ x, float* __restrict__ y,
                                                          float* __restrict__ var, size_t rows, float eps,
                                                          const float* __restrict__ w, float* __restrict__ out) {
  constexpr uint32_t axis = 128 * NV;
  const size_t row = (size_t)blockIdx.x * kHalfRowsPerBlock + threadIdx.x / 32;
  const int hl = threadIdx.x % 32;
  if (row >= rows) return;  // whole half-waves leave together
  const float4* xr = reinterpret_cast<const float4*>(x + row * axis);
  float v[4 * NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const float4 t = xr[hl + 32 * j];
    v[4 * j] = t.x; v[4 * j + 1] = t.y; v[4 * j + 2] = t.z; v[4 * j + 3] = t.w;
  }
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < 4 * NV; ++e) s += v[e];
  s = hsum(s);
  const float mu = s / (float)axis;
  float q = 0.0f;
#pragma unroll
  for (int e = 0; e < 4 * NV; ++e) { float dd = v[e] - mu; q += dd * dd; }
  q = hsum(q);
  const float va = q / (float)axis;
  const float sigma = sqrtf(va + eps);
#pragma unroll
  for (int e = 0; e < 4 * NV; ++e) v[e] = (v[e] - mu) / sigma;
  float4* yr = reinterpret_cast<float4*>(y + row * axis);
#pragma unroll
  for (int j = 0; j < NV; ++j) yr[hl + 32 * j] = make_float4(v[4 * j], v[4 * j + 1], v[4 * j + 2], v[4 * j + 3]);
  if (hl == 0 && var) var[row] = va;
  if (w) {
    const float4* wr = reinterpret_cast<const float4*>(w);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const float4 g = wr[hl + 32 * j];
      const float4 o = make_float4(v[4 * j] * g.x, v[4 * j + 1] * g.y, v[4 * j + 2] * g.z, v[4 * j + 3] * g.w);
      if constexpr (OB) {
        typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
        reinterpret_cast<bf16x4*>(reinterpret_cast<__bf16*>(out) + row * axis)[hl + 32 * j] =
            bf16x4{(__bf16)o.x, (__bf16)o.y, (__bf16)o.z, (__bf16)o.w};
      } else {
        reinterpret_cast<float4*>(out + row * axis)[hl + 32 * j] = o;
      }
    }
  }
}

template <int NV>
__global__ __launch_bounds__(256) void k_layernorm_bwd_rows32(const float* __restrict__ y, const float* __restrict__ var,
                                                              const float* __restrict__ dout, float* __restrict__ dx,
                                                              size_t rows, float eps, const float* __restrict__ addend,
                                                              const float* __restrict__ w) {
  constexpr uint32_t axis = 128 * NV;
  const size_t row = (size_t)blockIdx.x * kHalfRowsPerBlock + threadIdx.x / 32;
  const int hl = threadIdx.x % 32;
  if (row >= rows) return;
  const float4* yr = reinterpret_cast<const float4*>(y + row * axis);
  const float4* dr = reinterpret_cast<const float4*>(dout + row * axis);
  float yv[4 * NV], dv[4 * NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const float4 a = yr[hl + 32 * j], b = dr[hl + 32 * j];
    yv[4 * j] = a.x; yv[4 * j + 1] = a.y; yv[4 * j + 2] = a.z; yv[4 * j + 3] = a.w;
    dv[4 * j] = b.x; dv[4 * j + 1] = b.y; dv[4 * j + 2] = b.z; dv[4 * j + 3] = b.w;
  }
  if (w) {  // dout is the gradient of y * w: dy = dout * w, rounded like the multiply's VJP
    const float4* wr = reinterpret_cast<const float4*>(w);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const float4 g = wr[hl + 32 * j];
      dv[4 * j] = dv[4 * j] * g.x; dv[4 * j + 1] = dv[4 * j + 1] * g.y;
      dv[4 * j + 2] = dv[4 * j + 2] * g.z; dv[4 * j + 3] = dv[4 * j + 3] * g.w;
    }
  }
  float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
  for (int e = 0; e < 4 * NV; ++e) { s1 += dv[e]; float p = dv[e] * yv[e]; s2 += p; }
  s1 = hsum(s1);
  s2 = hsum(s2);
  const float dy_mean = s1 / (float)axis;
  const float dyy_mean = s2 / (float)axis;
  const float inv_sigma = 1.0f / sqrtf(var[row] + eps);
#pragma unroll
  for (int e = 0; e < 4 * NV; ++e) {
    float y_term = yv[e] * dyy_mean;
    float tmp = dv[e] - dy_mean;
    float numer = tmp - y_term;
    yv[e] = numer * inv_sigma;
  }
  if (addend) {  // gradient accumulation: old + this VJP's value
    const float4* ar = reinterpret_cast<const float4*>(addend + row * axis);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const float4 a = ar[hl + 32 * j];
      yv[4 * j] = a.x + yv[4 * j]; yv[4 * j + 1] = a.y + yv[4 * j + 1];
      yv[4 * j + 2] = a.z + yv[4 * j + 2]; yv[4 * j + 3] = a.w + yv[4 * j + 3];
    }
  }
  float4* xr = reinterpret_cast<float4*>(dx + row * axis);
#pragma unroll
  for (int j = 0; j < NV; ++j) xr[hl + 32 * j] = make_float4(yv[4 * j], yv[4 * j + 1], yv[4 * j + 2], yv[4 * j + 3]);
}

// k_layernorm_bwd_rows32 for the rows of one 32-row chunk per workgroup
// (half-wave h takes rows beg + h + 8 k, k = 0..3), which also forms the
// chunk's column partial of dw = sum over rows of dout * y (the scale's
// VJP): each half-wave sums its rows' products in k order, then the eight
// half-waves' sums are added in order.  That is exactly the partial the
// column reduction (k_col4 with 8 row-threads over 32-row chunks) writes,
// so the combined dw is the separate reduction's, bit for bit.  The
// partials go row-major, partial[chunk * axis + c] (one contiguous row per
// workgroup; the reduction's column-major layout, a 4-byte store per column
// at the stride of the chunk count, made this kernel 9 % slower at C5), and
// col_combine_sum adds them in the order the reduction's combine uses.
template <int NV>
__global__ __launch_bounds__(256) void k_layernorm_bwd_scale_rows32(const float* __restrict__ y,
                                                                    const float* __restrict__ var,
                                                                    const float* __restrict__ dout,
                                                                    float* __restrict__ dx, size_t rows, float eps,
                                                                    const float* __restrict__ addend,
                                                                    const float* __restrict__ w,
                                                                    float* __restrict__ partial, uint32_t nsplit) {
  constexpr uint32_t axis = 128 * NV;
  __shared__ float red[8][axis];
  const int hw = threadIdx.x / 32, hl = threadIdx.x % 32;
  float pacc[4 * NV];
#pragma unroll
  for (int e = 0; e < 4 * NV; ++e) pacc[e] = 0.0f;
#pragma unroll 1
  for (int k = 0; k < 4; ++k) {
    const size_t row = (size_t)blockIdx.x * 32 + hw + 8 * k;
    if (row >= rows) break;  // uniform over the half-wave
    const float4* yr = reinterpret_cast<const float4*>(y + row * axis);
    const float4* dr = reinterpret_cast<const float4*>(dout + row * axis);
    float yv[4 * NV], dv[4 * NV];
    float4 av[NV];  // the addend row, loaded with y and dout (one memory round trip per row)
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const float4 a = yr[hl + 32 * j], b = dr[hl + 32 * j];
      if (addend) av[j] = reinterpret_cast<const float4*>(addend + row * axis)[hl + 32 * j];
      yv[4 * j] = a.x; yv[4 * j + 1] = a.y; yv[4 * j + 2] = a.z; yv[4 * j + 3] = a.w;
      dv[4 * j] = b.x; dv[4 * j + 1] = b.y; dv[4 * j + 2] = b.z; dv[4 * j + 3] = b.w;
    }
#pragma unroll
    for (int e = 0; e < 4 * NV; ++e) {
      const float p = dv[e] * yv[e];  // dout * y, rounded like the reduction's product
      pacc[e] = pacc[e] + p;
    }
    const float4* wr = reinterpret_cast<const float4*>(w);
#pragma unroll
    for (int j = 0; j < NV; ++j) {
      const float4 g = wr[hl + 32 * j];
      dv[4 * j] = dv[4 * j] * g.x; dv[4 * j + 1] = dv[4 * j + 1] * g.y;
      dv[4 * j + 2] = dv[4 * j + 2] * g.z; dv[4 * j + 3] = dv[4 * j + 3] * g.w;
    }
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int e = 0; e < 4 * NV; ++e) { s1 += dv[e]; float p = dv[e] * yv[e]; s2 += p; }
    s1 = hsum(s1);
    s2 = hsum(s2);
    const float dy_mean = s1 / (float)axis;
    const float dyy_mean = s2 / (float)axis;
    const float inv_sigma = 1.0f / sqrtf(var[row] + eps);
#pragma unroll
    for (int e = 0; e < 4 * NV; ++e) {
      float y_term = yv[e] * dyy_mean;
      float tmp = dv[e] - dy_mean;
      float numer = tmp - y_term;
      yv[e] = numer * inv_sigma;
    }
    if (addend) {
#pragma unroll
      for (int j = 0; j < NV; ++j) {
        const float4 a = av[j];
        yv[4 * j] = a.x + yv[4 * j]; yv[4 * j + 1] = a.y + yv[4 * j + 1];
        yv[4 * j + 2] = a.z + yv[4 * j + 2]; yv[4 * j + 3] = a.w + yv[4 * j + 3];
      }
    }
    float4* xr = reinterpret_cast<float4*>(dx + row * axis);
#pragma unroll
    for (int j = 0; j < NV; ++j) xr[hl + 32 * j] = make_float4(yv[4 * j], yv[4 * j + 1], yv[4 * j + 2], yv[4 * j + 3]);
  }
#pragma unroll
  for (int j = 0; j < NV; ++j)
#pragma unroll
    for (int c = 0; c < 4; ++c) red[hw][4 * (hl + 32 * j) + c] = pacc[4 * j + c];
  __syncthreads();
  for (uint32_t col = threadIdx.x; col < axis; col += 256) {
    float r = red[0][col];
#pragma unroll
    for (int h = 1; h < 8; ++h) r = r + red[h][col];
    partial[(size_t)blockIdx.x * axis + col] = r;
  }
}

// cross_entropy.ml:18-28 / metal.rs:1555-1598: probs = softmax(logits, 1),
// nll[i] = -log(probs[i, t_i]) read back from the rounded probability.
template <int NV, int VM>
__global__ __launch_bounds__(256) void k_ce_fwd_rows(const float* __restrict__ logits, const int32_t* __restrict__ tgt,
                                                     float* __restrict__ probs, float* __restrict__ nll, size_t rows,
                                                     uint32_t axis, int32_t* __restrict__ err) {
  const size_t row = (size_t)blockIdx.x * kRowsPerBlock + threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  if (row >= rows) return;
  const int32_t tg = tgt[row];  // issued with the row's loads
  RowTile<NV, VM> t;
  t.load(logits + row * axis, axis, lane, -INFINITY);
  float m = -INFINITY;
#pragma unroll
  for (int e = 0; e < NV * 4; ++e) m = fmaxf(m, t.v[e]);
  m = wmax(m);
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < NV * 4; ++e) {
    float ex = t.valid(e, lane, axis) ? expf(t.v[e] - m) : 0.0f;
    t.v[e] = ex;
    s += ex;
  }
  s = wsum(s);
#pragma unroll
  for (int e = 0; e < NV * 4; ++e) t.v[e] = t.v[e] / s;
  t.store(probs + row * axis, axis, lane);
  if (tg < 0 || (uint32_t)tg >= axis) {
    if (lane == 0) { nll[row] = NAN; *err = 2; }
    return;
  }
  // the lane holding column tg takes the one log (integer compare: exact)
  float pt = 0.0f;
  bool own = false;
#pragma unroll
  for (int e = 0; e < NV * 4; ++e)
    if (t.col(e, lane) == (uint32_t)tg) { pt = t.v[e]; own = true; }
  if (own) nll[row] = -logf(pt);
}

// transformer_bwd.ml:57-65 / tape.rs:1200-1214: (p - 1{j == t}) * (dout[0] / N)
__global__ __launch_bounds__(256) void k_ce_bwd(const float* __restrict__ probs, const int32_t* __restrict__ tgt,
                                                const float* __restrict__ dout, float scale_host, float* __restrict__ dx,
                                                size_t n, uint32_t v) {
  const float scale = dout ? dout[0] / (float)n : scale_host;
  const size_t total = n * v, stride = (size_t)gridDim.x * blockDim.x;
  for (size_t f = (size_t)blockIdx.x * blockDim.x + threadIdx.x; f < total; f += stride) {
    size_t i = f / v;
    uint32_t j = (uint32_t)(f % v);
    float g = probs[f];
    if ((int32_t)j == tgt[i]) g = g - 1.0f;
    dx[f] = g * scale;
  }
}

// Same expression, four consecutive columns of one row per thread (v % 4 == 0,
// fewer than 2^32 elements): 32-bit index math, non-temporal streaming.
__global__ __launch_bounds__(256) void k_ce_bwd4(const float* __restrict__ probs, const int32_t* __restrict__ tgt,
                                                 const float* __restrict__ dout, float scale_host, float* __restrict__ dx,
                                                 uint32_t n, uint32_t v, uint32_t total4) {
  const float scale = dout ? dout[0] / (float)n : scale_host;
  const uint32_t stride = gridDim.x * blockDim.x;
  for (uint32_t f4 = blockIdx.x * blockDim.x + threadIdx.x; f4 < total4; f4 += stride) {
    const uint32_t f = 4 * f4, i = f / v, j = f - i * v;
    const int32_t t = tgt[i];
    const v4f p = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(probs) + f4);
    float g0 = p.x, g1 = p.y, g2 = p.z, g3 = p.w;
    if ((int32_t)j == t) g0 = g0 - 1.0f;
    if ((int32_t)(j + 1) == t) g1 = g1 - 1.0f;
    if ((int32_t)(j + 2) == t) g2 = g2 - 1.0f;
    if ((int32_t)(j + 3) == t) g3 = g3 - 1.0f;
    __builtin_nontemporal_store(v4f{g0 * scale, g1 * scale, g2 * scale, g3 * scale}, reinterpret_cast<v4f*>(dx) + f4);
  }
}

__global__ __launch_bounds__(256) void k_nll_gather(const float* __restrict__ probs, const int32_t* __restrict__ tgt,
                                                    float* __restrict__ nll, size_t n, uint32_t v, int32_t* __restrict__ err) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  int32_t t = tgt[i];
  if (t < 0 || (uint32_t)t >= v) { nll[i] = NAN; *err = 2; return; }
  nll[i] = -logf(probs[i * v + (uint32_t)t]);
}

// ---- sequential fallbacks: one thread per (outer, inner) ------------------
__global__ void k_softmax_seq(const float* __restrict__ x, float* __restrict__ y, size_t outer, size_t axis, size_t inner) {
  size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= outer * inner) return;
  size_t o = id / inner, i = id % inner;
  const float* xb = x + o * axis * inner + i;
  float* yb = y + o * axis * inner + i;
  float mx = -INFINITY;
  for (size_t k = 0; k < axis; ++k) if (xb[k * inner] > mx) mx = xb[k * inner];
  float sum = 0.0f;
  for (size_t k = 0; k < axis; ++k) { float e = expf(xb[k * inner] - mx); yb[k * inner] = e; sum += e; }
  for (size_t k = 0; k < axis; ++k) yb[k * inner] = yb[k * inner] / sum;
}

__global__ void k_softmax_bwd_seq(const float* __restrict__ s, const float* __restrict__ d, float* __restrict__ dx,
                                  size_t outer, size_t axis, size_t inner) {
  size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= outer * inner) return;
  size_t base = (id / inner) * axis * inner + id % inner;
  float acc = 0.0f;
  for (size_t k = 0; k < axis; ++k) { float p = d[base + k * inner] * s[base + k * inner]; acc += p; }
  for (size_t k = 0; k < axis; ++k) { float diff = d[base + k * inner] - acc; dx[base + k * inner] = s[base + k * inner] * diff; }
}

__global__ void k_layernorm_seq(const float* __restrict__ x, float* __restrict__ y, float* __restrict__ var, size_t outer,
                                size_t axis, size_t inner, float eps) {
  size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= outer * inner) return;
  size_t base = (id / inner) * axis * inner + id % inner;
  float mu = 0.0f;
  for (size_t k = 0; k < axis; ++k) mu += x[base + k * inner];
  mu = mu / (float)axis;
  float va = 0.0f;
  for (size_t k = 0; k < axis; ++k) { float d = x[base + k * inner] - mu; va += d * d; }
  va = va / (float)axis;
  float sigma = sqrtf(va + eps);
  if (var) var[id] = va;
  for (size_t k = 0; k < axis; ++k) y[base + k * inner] = (x[base + k * inner] - mu) / sigma;
}

__global__ void k_layernorm_bwd_seq(const float* __restrict__ y, const float* __restrict__ var, const float* __restrict__ d,
                                    float* __restrict__ dx, size_t outer, size_t axis, size_t inner, float eps) {
  size_t id = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (id >= outer * inner) return;
  size_t base = (id / inner) * axis * inner + id % inner;
  float inv_sigma = 1.0f / sqrtf(var[id] + eps);
  float s1 = 0.0f, s2 = 0.0f;
  for (size_t k = 0; k < axis; ++k) s1 += d[base + k * inner];
  for (size_t k = 0; k < axis; ++k) { float p = d[base + k * inner] * y[base + k * inner]; s2 += p; }
  float dym = s1 / (float)axis, dyym = s2 / (float)axis;
  for (size_t k = 0; k < axis; ++k) {
    float y_term = y[base + k * inner] * dyym;
    float tmp = d[base + k * inner] - dym;
    float numer = tmp - y_term;
    dx[base + k * inner] = numer * inv_sigma;
  }
}

__global__ void k_ce_fwd_seq(const float* __restrict__ logits, const int32_t* __restrict__ tgt, float* __restrict__ probs,
                             float* __restrict__ nll, size_t n, size_t v, int32_t* __restrict__ err) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float* x = logits + i * v;
  float* p = probs + i * v;
  float mx = -INFINITY;
  for (size_t k = 0; k < v; ++k) if (x[k] > mx) mx = x[k];
  float sum = 0.0f;
  for (size_t k = 0; k < v; ++k) { float e = expf(x[k] - mx); p[k] = e; sum += e; }
  for (size_t k = 0; k < v; ++k) p[k] = p[k] / sum;
  int32_t t = tgt[i];
  if (t < 0 || (size_t)t >= v) { nll[i] = NAN; *err = 2; return; }
  nll[i] = -logf(p[t]);
}

// Launch helper: choose the register-tile width for a row length.
// Stream with non-temporal loads when an op's operands exceed the 256 MB
// last-level cache (measured: ~+15 % on [65536, 1024] rows; on the training
// step's <= 100 MB operands cached loads are faster).
constexpr size_t kStreamBytes = 256ull << 20;

template <template <int, int> class KSel, class Launch>
void row_dispatch(uint32_t axis, Launch launch, size_t bytes = 0) {
  const bool vec = (axis % 4) == 0;
  const bool nt = bytes >= kStreamBytes;
  // elements per lane needed: ceil(axis / 64)
  uint32_t per_lane = (axis + 63) / 64;
  int nv = per_lane <= 4 ? 1 : per_lane <= 8 ? 2 : per_lane <= 16 ? 4 : per_lane <= 32 ? 8 : 16;
#define MALUS_ROW_CASE(NV)                                       \
  case NV:                                                       \
    if (vec && nt) launch(KSel<NV, 2>{});                             \
    else if (vec) launch(KSel<NV, 1>{});                             \
    else launch(KSel<NV, 0>{});                                      \
    break;
  switch (nv) {
    MALUS_ROW_CASE(1)
    MALUS_ROW_CASE(2)
    MALUS_ROW_CASE(4)
    MALUS_ROW_CASE(8)
    MALUS_ROW_CASE(16)
  }
#undef MALUS_ROW_CASE
}

template <int NV, int VM> struct SelSoftmax { static constexpr auto fn = k_softmax_rows<NV, VM>; };
template <int NV, int VM> struct SelSoftmaxBwd { static constexpr auto fn = k_softmax_bwd_rows<NV, VM>; };
template <int NV, int VM> struct SelScaleMaskSoftmax { static constexpr auto fn = k_scale_mask_softmax_rows<NV, VM>; };
template <int NV, int VM> struct SelLN { static constexpr auto fn = k_layernorm_rows<NV, VM>; };
template <int NV, int VM> struct SelLNBwd { static constexpr auto fn = k_layernorm_bwd_rows<NV, VM>; };
template <int NV, int VM> struct SelCE { static constexpr auto fn = k_ce_fwd_rows<NV, VM>; };

constexpr uint32_t kMaxRowAxis = 4096;
inline unsigned row_grid(size_t rows) { return (unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock); }
inline unsigned seq_grid(size_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

void softmax(const float* x, float* out, size_t outer, size_t axis, size_t inner, hipStream_t s) {
  if (!outer || !axis || !inner) return;
  if (inner == 1 && axis <= kMaxRowAxis) {
    row_dispatch<SelSoftmax>((uint32_t)axis, [&](auto sel) {
      decltype(sel)::fn<<<row_grid(outer), 256, 0, s>>>(x, out, outer, (uint32_t)axis);
    }, 2 * outer * (size_t)axis * sizeof(float));
  } else {
    k_softmax_seq<<<seq_grid(outer * inner), 256, 0, s>>>(x, out, outer, axis, inner);
  }
  MALUS_HIP(hipGetLastError());
}

void scale_mask_softmax(const float* S, const float* scale, const float* mask, float* P, size_t rows, size_t axis,
                        size_t mask_rows, hipStream_t s) {
  if (!rows || !axis) return;
  if (axis <= kMaxRowAxis && mask_rows > 0) {
    row_dispatch<SelScaleMaskSoftmax>((uint32_t)axis, [&](auto sel) {
      decltype(sel)::fn<<<row_grid(rows), 256, 0, s>>>(S, scale, mask, P, rows, (uint32_t)axis, (uint32_t)mask_rows);
    }, 2 * rows * (size_t)axis * sizeof(float));
    MALUS_HIP(hipGetLastError());
    return;
  }
  // wide rows: the three separate kernels through a temporary
  const size_t n = rows * axis;
  size_t bucket;
  float* tmp = static_cast<float*>(pool_alloc(n * sizeof(float), &bucket));
  binary_scalar(MUL, S, scale, 0.0f, true, tmp, n, s);
  binary_rowbcast(ADD, tmp, mask, tmp, n, mask_rows * axis, s);
  softmax(tmp, P, rows, axis, 1, s);
  pool_free(tmp, bucket);
}

void softmax_bwd(const float* y, const float* dout, float* out, size_t outer, size_t axis, size_t inner, hipStream_t s) {
  if (!outer || !axis || !inner) return;
  if (inner == 1 && axis <= kMaxRowAxis) {
    row_dispatch<SelSoftmaxBwd>((uint32_t)axis, [&](auto sel) {
      decltype(sel)::fn<<<row_grid(outer), 256, 0, s>>>(y, dout, out, outer, (uint32_t)axis);
    }, 3 * outer * (size_t)axis * sizeof(float));
  } else {
    k_softmax_bwd_seq<<<seq_grid(outer * inner), 256, 0, s>>>(y, dout, out, outer, axis, inner);
  }
  MALUS_HIP(hipGetLastError());
}

void layernorm(const float* x, float* y, float* var, size_t outer, size_t axis, size_t inner, float eps, hipStream_t s,
               const float* w, float* out, bool out_bf16) {
  if (!outer || !axis || !inner) return;
  const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const bool rows32 = inner == 1 && axis % 128 == 0 && axis <= 512 && a16(x) && a16(y) && a16(w) && a16(out);
  if (out_bf16) {
    if (!rows32 || !w) fail("malus: layernorm: a bf16 affine output needs the last axis, a multiple of 128 up to 512");
    const unsigned grid = (unsigned)((outer + kHalfRowsPerBlock - 1) / kHalfRowsPerBlock);
    switch (axis / 128) {
      case 1: k_layernorm_rows32<1, true><<<grid, 256, 0, s>>>(x, y, var, outer, eps, w, out); break;
      case 2: k_layernorm_rows32<2, true><<<grid, 256, 0, s>>>(x, y, var, outer, eps, w, out); break;
      case 3: k_layernorm_rows32<3, true><<<grid, 256, 0, s>>>(x, y, var, outer, eps, w, out); break;
      default: k_layernorm_rows32<4, true><<<grid, 256, 0, s>>>(x, y, var, outer, eps, w, out); break;
    }
  } else if (rows32) {
    const unsigned grid = (unsigned)((outer + kHalfRowsPerBlock - 1) / kHalfRowsPerBlock);
    switch (axis / 128) {
      case 1: k_layernorm_rows32<1><<<grid, 256, 0, s>>>(x, y, var, outer, eps, w, out); break;
      case 2: k_layernorm_rows32<2><<<grid, 256, 0, s>>>(x, y, var, outer, eps, w, out); break;
      case 3: k_layernorm_rows32<3><<<grid, 256, 0, s>>>(x, y, var, outer, eps, w, out); break;
      default: k_layernorm_rows32<4><<<grid, 256, 0, s>>>(x, y, var, outer, eps, w, out); break;
    }
  } else if (inner == 1 && axis <= kMaxRowAxis) {
    row_dispatch<SelLN>((uint32_t)axis, [&](auto sel) {
      decltype(sel)::fn<<<row_grid(outer), 256, 0, s>>>(x, y, var, outer, (uint32_t)axis, eps, w, out);
    }, (w ? 3 : 2) * outer * (size_t)axis * sizeof(float));
  } else {
    if (w) fail("malus: fused layernorm scale needs the normalized axis last");
    k_layernorm_seq<<<seq_grid(outer * inner), 256, 0, s>>>(x, y, var, outer, axis, inner, eps);
  }
  MALUS_HIP(hipGetLastError());
}

void layernorm_bwd(const float* y, const float* var, const float* dout, float* dx, size_t outer, size_t axis, size_t inner,
                   float eps, hipStream_t s, const float* addend, const float* w) {
  if (!outer || !axis || !inner) return;
  const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (inner == 1 && axis % 128 == 0 && axis <= 512 && a16(y) && a16(dout) && a16(dx) && a16(addend) && a16(w)) {
    const unsigned grid = (unsigned)((outer + kHalfRowsPerBlock - 1) / kHalfRowsPerBlock);
    switch (axis / 128) {
      case 1: k_layernorm_bwd_rows32<1><<<grid, 256, 0, s>>>(y, var, dout, dx, outer, eps, addend, w); break;
      case 2: k_layernorm_bwd_rows32<2><<<grid, 256, 0, s>>>(y, var, dout, dx, outer, eps, addend, w); break;
      case 3: k_layernorm_bwd_rows32<3><<<grid, 256, 0, s>>>(y, var, dout, dx, outer, eps, addend, w); break;
      default: k_layernorm_bwd_rows32<4><<<grid, 256, 0, s>>>(y, var, dout, dx, outer, eps, addend, w); break;
    }
  } else if (inner == 1 && axis <= kMaxRowAxis) {
    row_dispatch<SelLNBwd>((uint32_t)axis, [&](auto sel) {
      decltype(sel)::fn<<<row_grid(outer), 256, 0, s>>>(y, var, dout, dx, outer, (uint32_t)axis, eps, addend, w);
    }, 3 * outer * (size_t)axis * sizeof(float));
  } else {
    if (w) fail("malus: fused layernorm scale needs the normalized axis last");
    k_layernorm_bwd_seq<<<seq_grid(outer * inner), 256, 0, s>>>(y, var, dout, dx, outer, axis, inner, eps);
    if (addend) binary_same(ADD, addend, dx, dx, outer * axis * inner, s);
  }
  MALUS_HIP(hipGetLastError());
}

bool layernorm_bwd_scale(const float* y, const float* var, const float* dout, float* dx, float* dw, size_t rows,
                         size_t axis, float eps, hipStream_t s, const float* addend, const float* w, bool defer_dw) {
  const auto a16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (!rows || axis % 128 != 0 || axis > 512 || !w || !a16(y) || !a16(dout) || !a16(dx) || !a16(addend) || !a16(w))
    return false;
  uint32_t nsplit = 0;
  size_t chunk = 0;
  int rt = 0;
  // the chunking must be the one the separate column reduction uses
  if (!col_prod_split(rows, axis, &nsplit, &chunk, &rt) || chunk != 32 || rt != 8) return false;
  size_t bucket;
  float* partial = static_cast<float*>(pool_alloc(axis * nsplit * sizeof(float), &bucket));
  switch (axis / 128) {
    case 1: k_layernorm_bwd_scale_rows32<1><<<nsplit, 256, 0, s>>>(y, var, dout, dx, rows, eps, addend, w, partial, nsplit); break;
    case 2: k_layernorm_bwd_scale_rows32<2><<<nsplit, 256, 0, s>>>(y, var, dout, dx, rows, eps, addend, w, partial, nsplit); break;
    case 3: k_layernorm_bwd_scale_rows32<3><<<nsplit, 256, 0, s>>>(y, var, dout, dx, rows, eps, addend, w, partial, nsplit); break;
    default: k_layernorm_bwd_scale_rows32<4><<<nsplit, 256, 0, s>>>(y, var, dout, dx, rows, eps, addend, w, partial, nsplit); break;
  }
  MALUS_HIP(hipGetLastError());
  col_combine_sum_owned(partial, bucket, dw, axis, nsplit, rows, defer_dw, s);
  return true;
}

void ce_fwd(const float* logits, const int32_t* tgt, float* probs, float* nll, size_t n, size_t v, int32_t* err,
            hipStream_t s) {
  if (!n || !v) return;
  if (v <= kMaxRowAxis) {
    row_dispatch<SelCE>((uint32_t)v, [&](auto sel) {
      decltype(sel)::fn<<<row_grid(n), 256, 0, s>>>(logits, tgt, probs, nll, n, (uint32_t)v, err);
    }, 2 * n * (size_t)v * sizeof(float));
  } else {
    k_ce_fwd_seq<<<seq_grid(n), 256, 0, s>>>(logits, tgt, probs, nll, n, v, err);
  }
  MALUS_HIP(hipGetLastError());
}

void ce_bwd(const float* probs, const int32_t* tgt, const float* dout, float scale_host, float* dx, size_t n, size_t v,
            hipStream_t s) {
  size_t total = n * v;
  if (!total) return;
  if (v % 4 == 0 && total < (1ull << 32)) {
    const size_t total4 = total / 4;
    size_t blocks = (total4 + 255) / 256;
    if (blocks > (1u << 20)) blocks = 1u << 20;
    k_ce_bwd4<<<(unsigned)blocks, 256, 0, s>>>(probs, tgt, dout, scale_host, dx, (uint32_t)n, (uint32_t)v, (uint32_t)total4);
    MALUS_HIP(hipGetLastError());
    return;
  }
  size_t blocks = (total + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  k_ce_bwd<<<(unsigned)blocks, 256, 0, s>>>(probs, tgt, dout, scale_host, dx, n, (uint32_t)v);
  MALUS_HIP(hipGetLastError());
}

void nll_gather(const float* probs, const int32_t* tgt, float* nll, size_t n, size_t v, int32_t* err, hipStream_t s) {
  if (!n) return;
  k_nll_gather<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(probs, tgt, nll, n, (uint32_t)v, err);
  MALUS_HIP(hipGetLastError());
}

}  // namespace k
}  // namespace malus
