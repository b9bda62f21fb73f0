// Elementwise kernels for gfx950: broadcast binops, scalar binops, unary
// builtins and their VJPs, fills.  HBM-bound: 128-bit non-temporal loads and
// stores of the streamed operands (broadcast rows stay cached), four float4
// chunks per thread with the grid sized to cover the tensor in one pass
// (a grid-stride loop only past 2^20 workgroups), and a scalar tail.  Built
// with -ffp-contract=off so every expression rounds like the reference's
// one-op-per-kernel f32 arithmetic.
#include "common.h"
#include "k_gelu.h"
#include "k_split.h"

namespace malus {
namespace k {
namespace {

constexpr int kBlock = 256;
constexpr int kEwUnroll = 2;  // float4 chunks per thread

inline unsigned ew_grid(size_t work_items) {
  // kEwUnroll float4 chunks per thread: one pass over the tensor (measured
  // on gfx950 at 2^26 f32: a single pass with non-temporal access beats a
  // capped grid-stride loop by ~25 %; two chunks per thread stream 2-4
  // points of HBM peak faster than four or eight, and one loses 9 points on
  // GELU's arithmetic).
  size_t blocks = (work_items + kBlock * kEwUnroll - 1) / (kBlock * kEwUnroll);
  if (blocks < 1) blocks = 1;
  if (blocks > (1u << 20)) blocks = 1u << 20;
  return (unsigned)blocks;
}

template <int OP>
__device__ __forceinline__ float binop(float a, float b) {
  if constexpr (OP == ADD) return a + b;
  else if constexpr (OP == SUB) return a - b;
  else if constexpr (OP == MUL) return a * b;
  else return a / b;
}

// Unary builtins: codegen-gpu/lib.rs:375-381; GELU: metal.rs:1535-1549.
// exp / log / tanh are evaluated in f64 and rounded once to f32, so each is
// within 0.5 ulp (+ a rare double-rounding step) of the exact value, like
// the host libm the reference's CPU path calls; the f32 device library is
// up to ~4 ulp off at large |x|.  These kernels are HBM-bound, so the f64
// arithmetic is hidden behind the memory traffic.
template <int OP>
__device__ __forceinline__ float unop(float x) {
  if constexpr (OP == RELU) return fmaxf(0.0f, x);
  else if constexpr (OP == SIGMOID) return 1.0f / (1.0f + (float)exp(-(double)x));
  else if constexpr (OP == TANH) return (float)tanh((double)x);
  else if constexpr (OP == EXP) return (float)exp((double)x);
  else if constexpr (OP == LOG) return (float)log((double)x);
  else if constexpr (OP == SQRT) return sqrtf(x);
  else if constexpr (OP == ABS) return fabsf(x);
  else return gelu_fwd(x);  // tanh approximation (k_gelu.h)
}

// Unary VJPs: tape.rs:1041-1083 and 1187-1199 (expression order kept).
template <int OP>
__device__ __forceinline__ float unbwd(float v, float d) {
  if constexpr (OP == B_SIGMOID) { float t = d * v; float oms = 1.0f - v; return t * oms; }
  else if constexpr (OP == B_RELU) return d * (v > 0.0f ? 1.0f : 0.0f);
  else if constexpr (OP == B_TANH) return d * (1.0f - v * v);
  else if constexpr (OP == B_SQRT) { float two_s = v * 2.0f; return d / two_s; }
  else if constexpr (OP == B_ABS) return d * (v > 0.0f ? 1.0f : (v < 0.0f ? -1.0f : 0.0f));
  else if constexpr (OP == B_EXP) return d * v;
  else if constexpr (OP == B_LOG) return d / v;
  else return gelu_bwd(v, d);  // B_GELU (k_gelu.h)
}

typedef float v4f __attribute__((ext_vector_type(4)));
// Streamed operands: non-temporal 128-bit access (each byte is touched once).
__device__ __forceinline__ float4 ld4(const float* p, size_t i) {
  const v4f v = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(p) + i);
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st4(float* p, size_t i, float4 v) {
  __builtin_nontemporal_store(v4f{v.x, v.y, v.z, v.w}, reinterpret_cast<v4f*>(p) + i);
}
// Broadcast operands (re-read by many threads): ordinary cached loads.
__device__ __forceinline__ float4 ld4c(const float* p, size_t i) { return reinterpret_cast<const float4*>(p)[i]; }

// Generic float4 grid-stride driver: F(i4) produces output chunk i4, and
// T(i) produces scalar element i for the tail.
template <class F4, class F1>
__device__ __forceinline__ void ew_loop(size_t n, float* out, F4 f4, F1 f1) {
  const size_t n4 = n >> 2;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i + (kEwUnroll - 1) * stride < n4; i += kEwUnroll * stride) {
    float4 r[kEwUnroll];
#pragma unroll
    for (int u = 0; u < kEwUnroll; ++u) r[u] = f4(i + u * stride);
#pragma unroll
    for (int u = 0; u < kEwUnroll; ++u) st4(out, i + u * stride, r[u]);
  }
  for (; i < n4; i += stride) st4(out, i, f4(i));
  size_t t = (n4 << 2) + (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; t < n; t += stride) out[t] = f1(t);
}

template <int OP>
__global__ __launch_bounds__(kBlock) void k_binary_same(const float* __restrict__ p, const float* __restrict__ q,
                                                        float* __restrict__ out, size_t n) {
  ew_loop(n, out,
          [&](size_t i) {
            float4 a = ld4(p, i), b = ld4(q, i);
            return make_float4(binop<OP>(a.x, b.x), binop<OP>(a.y, b.y), binop<OP>(a.z, b.z), binop<OP>(a.w, b.w));
          },
          [&](size_t i) { return binop<OP>(p[i], q[i]); });
}

// q broadcast along leading dims: q index = i % qn (qn % 4 == 0 for the float4 path).
template <int OP>
__global__ __launch_bounds__(kBlock) void k_binary_rowb(const float* __restrict__ p, const float* __restrict__ q,
                                                        float* __restrict__ out, size_t n, uint32_t qn4) {
  ew_loop(n, out,
          [&](size_t i) {
            float4 a = ld4(p, i), b = ld4c(q, (uint32_t)(i % qn4));
            return make_float4(binop<OP>(a.x, b.x), binop<OP>(a.y, b.y), binop<OP>(a.z, b.z), binop<OP>(a.w, b.w));
          },
          [&](size_t i) { return binop<OP>(p[i], q[i % ((size_t)qn4 * 4)]); });
}

template <int OP>
__global__ __launch_bounds__(kBlock) void k_binary_rowb_scalar(const float* __restrict__ p, const float* __restrict__ q,
                                                               float* __restrict__ out, size_t n, size_t qn) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) out[i] = binop<OP>(p[i], q[i % qn]);
}

// p broadcast along leading dims (the higher-rank operand is q).
template <int OP>
__global__ __launch_bounds__(kBlock) void k_binary_rowb_rev(const float* __restrict__ p, const float* __restrict__ q,
                                                            float* __restrict__ out, size_t n, size_t pn) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) out[i] = binop<OP>(p[i % pn], q[i]);
}

template <int OP, bool RIGHT>
__global__ __launch_bounds__(kBlock) void k_binary_scalar(const float* __restrict__ p, const float* __restrict__ qdev,
                                                          float qval, float* __restrict__ out, size_t n) {
  const float s = qdev ? qdev[0] : qval;
  ew_loop(n, out,
          [&](size_t i) {
            float4 a = ld4(p, i);
            if constexpr (RIGHT)
              return make_float4(binop<OP>(a.x, s), binop<OP>(a.y, s), binop<OP>(a.z, s), binop<OP>(a.w, s));
            else
              return make_float4(binop<OP>(s, a.x), binop<OP>(s, a.y), binop<OP>(s, a.z), binop<OP>(s, a.w));
          },
          [&](size_t i) { return RIGHT ? binop<OP>(p[i], s) : binop<OP>(s, p[i]); });
}

template <int OP>
__global__ __launch_bounds__(kBlock) void k_binary_general(const float* __restrict__ p, const float* __restrict__ q,
                                                           float* __restrict__ out, size_t n, BcastDesc d) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    size_t rem = i, pf = 0, qf = 0;
    for (int dd = d.ndim - 1; dd >= 0; --dd) {
      size_t id = rem % d.out_shape[dd];
      rem /= d.out_shape[dd];
      pf += id * d.p_stride[dd];
      qf += id * d.q_stride[dd];
    }
    out[i] = binop<OP>(p[pf], q[qf]);
  }
}

template <int OP>
__global__ __launch_bounds__(kBlock) void k_unary(const float* __restrict__ x, float* __restrict__ out, size_t n) {
  ew_loop(n, out,
          [&](size_t i) {
            float4 a = ld4(x, i);
            return make_float4(unop<OP>(a.x), unop<OP>(a.y), unop<OP>(a.z), unop<OP>(a.w));
          },
          [&](size_t i) { return unop<OP>(x[i]); });
}

template <int OP>
__global__ __launch_bounds__(kBlock) void k_unary_bwd(const float* __restrict__ xy, const float* __restrict__ dout,
                                                      float* __restrict__ out, size_t n) {
  ew_loop(n, out,
          [&](size_t i) {
            float4 a = ld4(xy, i), d = ld4(dout, i);
            return make_float4(unbwd<OP>(a.x, d.x), unbwd<OP>(a.y, d.y), unbwd<OP>(a.z, d.z), unbwd<OP>(a.w, d.w));
          },
          [&](size_t i) { return unbwd<OP>(xy[i], dout[i]); });
}

__global__ __launch_bounds__(kBlock) void k_fill(float* __restrict__ out, float v, const float* __restrict__ vdev, size_t n) {
  const float s = vdev ? vdev[0] : v;
  ew_loop(n, out, [&](size_t) { return make_float4(s, s, s, s); }, [&](size_t) { return s; });
}

__global__ __launch_bounds__(kBlock) void k_eq(const float* __restrict__ a, const float* __restrict__ b,
                                               float* __restrict__ out, size_t n) {
  ew_loop(n, out,
          [&](size_t i) {
            float4 x = ld4(a, i), y = ld4(b, i);
            return make_float4(x.x == y.x ? 1.f : 0.f, x.y == y.y ? 1.f : 0.f, x.z == y.z ? 1.f : 0.f,
                               x.w == y.w ? 1.f : 0.f);
          },
          [&](size_t i) { return a[i] == b[i] ? 1.f : 0.f; });
}

// transformer_bwd.ml:6-8 (1/sqrt(v + eps) as the host VJP computes it, tape.rs:1164)
__global__ __launch_bounds__(kBlock) void k_rsqrt_eps(const float* __restrict__ v, float eps, float* __restrict__ out,
                                                      size_t n) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) out[i] = 1.0f / sqrtf(v[i] + eps);
}

__global__ __launch_bounds__(kBlock) void k_copy_bytes(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst,
                                                       size_t n16, size_t nbytes) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (size_t j = i; j < n16; j += stride)
    reinterpret_cast<uint4*>(dst)[j] = reinterpret_cast<const uint4*>(src)[j];
  for (size_t j = n16 * 16 + i; j < nbytes; j += stride) dst[j] = src[j];
}

__global__ __launch_bounds__(kBlock) void k_zero_bytes(uint8_t* __restrict__ dst, size_t n16, size_t nbytes) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (size_t j = i; j < n16; j += stride) reinterpret_cast<uint4*>(dst)[j] = make_uint4(0, 0, 0, 0);
  for (size_t j = n16 * 16 + i; j < nbytes; j += stride) dst[j] = 0;
}

// tensor_causal_mask, metal.rs:1600-1612: 0 on/below the diagonal, -1e9 above.
__global__ __launch_bounds__(kBlock) void k_causal_mask(float* __restrict__ out, uint32_t t) {
  size_t n = (size_t)t * t, stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    uint32_t r = (uint32_t)(i / t), c = (uint32_t)(i % t);
    out[i] = c > r ? -1e9f : 0.0f;
  }
}

__global__ __launch_bounds__(kBlock) void k_iota_rows(int32_t* __restrict__ out, size_t n, uint32_t t) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) out[i] = (int32_t)(i % t);
}

// f32 <-> bf16 conversions (the autocast storage type): to bf16 rounds to
// nearest even (NaN stays NaN), to f32 is exact.
__global__ __launch_bounds__(kBlock) void k_f32_to_bf16(const float* __restrict__ x, __bf16* __restrict__ out, size_t n) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) out[i] = (__bf16)x[i];
}
__global__ __launch_bounds__(kBlock) void k_bf16_to_f32(const __bf16* __restrict__ x, float* __restrict__ out, size_t n) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) out[i] = (float)x[i];
}

constexpr int kCvtMaxSegs = 64;
constexpr size_t kCvtChunk = 2048;  // elements per workgroup
struct CvtTable {
  Bf16Copy seg[kCvtMaxSegs];
  uint32_t first_chunk[kCvtMaxSegs + 1];
  int count;
};
static_assert(sizeof(CvtTable) + 64 <= 4096, "the segment table travels in the 4 KB of kernel arguments");
__global__ __launch_bounds__(kBlock) void k_to_bf16_multi(const CvtTable t) {
  int lo = 0, hi = t.count - 1;  // the segment holding chunk blockIdx.x
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (t.first_chunk[mid] <= blockIdx.x) lo = mid;
    else hi = mid - 1;
  }
  const Bf16Copy& sg = t.seg[lo];
  const size_t first = (size_t)(blockIdx.x - t.first_chunk[lo]) * kCvtChunk;
  const size_t end = first + kCvtChunk < sg.n ? first + kCvtChunk : sg.n;
  __bf16* dst = static_cast<__bf16*>(sg.dst);
  for (size_t i = first + threadIdx.x; i < end; i += blockDim.x) dst[i] = (__bf16)sg.src[i];
}

// The split copies: split3 (k_split.h) on runs of 8 values, so the pieces
// are the bits the split GEMM forms from the same values itself.  Chunks
// start at multiples of 8; a run cut short by the end of a tensor is
// padded with zeros and only its own values are stored.
__global__ __launch_bounds__(kBlock) void k_split3_multi(const CvtTable t) {
  int lo = 0, hi = t.count - 1;  // the segment holding chunk blockIdx.x
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (t.first_chunk[mid] <= blockIdx.x) lo = mid;
    else hi = mid - 1;
  }
  const Bf16Copy& sg = t.seg[lo];
  const size_t first = (size_t)(blockIdx.x - t.first_chunk[lo]) * kCvtChunk;
  const size_t end = first + kCvtChunk < sg.n ? first + kCvtChunk : sg.n;
  __bf16* ph = static_cast<__bf16*>(sg.dst);
  __bf16* pm = ph + sg.n;
  __bf16* pl = pm + sg.n;
  const bool vec = sg.n % 8 == 0 && ((reinterpret_cast<uintptr_t>(sg.src) | reinterpret_cast<uintptr_t>(sg.dst)) & 15) == 0;
  for (size_t i = first + 8 * (size_t)threadIdx.x; i < end; i += 8 * (size_t)blockDim.x) {
    float f[8];
    if (vec) {
      const float4 a = reinterpret_cast<const float4*>(sg.src + i)[0], b = reinterpret_cast<const float4*>(sg.src + i)[1];
      f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
      f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = i + e < end ? sg.src[i + e] : 0.0f;
    }
    const Split3 p = split3(f);
    if (vec) {
      *reinterpret_cast<bf16x8*>(ph + i) = p.h;
      *reinterpret_cast<bf16x8*>(pm + i) = p.m;
      *reinterpret_cast<bf16x8*>(pl + i) = p.l;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (i + e < end) {
          ph[i + e] = p.h[e];
          pm[i + e] = p.m[e];
          pl[i + e] = p.l[e];
        }
    }
  }
}

template <class F>
void dispatch_binop(int op, F f) {
  switch (op) {
    case ADD: f(std::integral_constant<int, ADD>{}); break;
    case SUB: f(std::integral_constant<int, SUB>{}); break;
    case MUL: f(std::integral_constant<int, MUL>{}); break;
    case DIV: f(std::integral_constant<int, DIV>{}); break;
    default: fail("malus: bad binop %d", op);
  }
}

inline void post_launch(const char* name) { MALUS_HIP(hipGetLastError()); (void)name; }

}  // namespace

void binary_same(int op, const float* p, const float* q, float* out, size_t n, hipStream_t s) {
  if (!n) return;
  dispatch_binop(op, [&](auto o) { k_binary_same<decltype(o)::value><<<ew_grid(n / 4 + 1), kBlock, 0, s>>>(p, q, out, n); });
  post_launch("binary_same");
}

void binary_rowbcast(int op, const float* p, const float* q, float* out, size_t n, size_t qn, hipStream_t s) {
  if (!n) return;
  if (qn % 4 == 0 && n % 4 == 0 && qn / 4 < (1u << 31)) {
    dispatch_binop(op, [&](auto o) {
      k_binary_rowb<decltype(o)::value><<<ew_grid(n / 4 + 1), kBlock, 0, s>>>(p, q, out, n, (uint32_t)(qn / 4));
    });
  } else {
    dispatch_binop(op, [&](auto o) {
      k_binary_rowb_scalar<decltype(o)::value><<<ew_grid(n), kBlock, 0, s>>>(p, q, out, n, qn);
    });
  }
  post_launch("binary_rowbcast");
}

void binary_rowbcast_rev(int op, const float* p, size_t pn, const float* q, float* out, size_t n, hipStream_t s) {
  if (!n) return;
  dispatch_binop(op, [&](auto o) { k_binary_rowb_rev<decltype(o)::value><<<ew_grid(n), kBlock, 0, s>>>(p, q, out, n, pn); });
  post_launch("binary_rowbcast_rev");
}

void binary_scalar(int op, const float* p, const float* qdev, float qval, bool right, float* out, size_t n, hipStream_t s) {
  if (!n) return;
  dispatch_binop(op, [&](auto o) {
    constexpr int O = decltype(o)::value;
    if (right) k_binary_scalar<O, true><<<ew_grid(n / 4 + 1), kBlock, 0, s>>>(p, qdev, qval, out, n);
    else k_binary_scalar<O, false><<<ew_grid(n / 4 + 1), kBlock, 0, s>>>(p, qdev, qval, out, n);
  });
  post_launch("binary_scalar");
}

void binary_general(int op, const float* p, const float* q, float* out, size_t n, const BcastDesc& d, hipStream_t s) {
  if (!n) return;
  dispatch_binop(op, [&](auto o) { k_binary_general<decltype(o)::value><<<ew_grid(n), kBlock, 0, s>>>(p, q, out, n, d); });
  post_launch("binary_general");
}

void unary(int op, const float* x, float* out, size_t n, hipStream_t s) {
  if (!n) return;
  unsigned g = ew_grid(n / 4 + 1);
  switch (op) {
    case RELU: k_unary<RELU><<<g, kBlock, 0, s>>>(x, out, n); break;
    case SIGMOID: k_unary<SIGMOID><<<g, kBlock, 0, s>>>(x, out, n); break;
    case TANH: k_unary<TANH><<<g, kBlock, 0, s>>>(x, out, n); break;
    case EXP: k_unary<EXP><<<g, kBlock, 0, s>>>(x, out, n); break;
    case LOG: k_unary<LOG><<<g, kBlock, 0, s>>>(x, out, n); break;
    case SQRT: k_unary<SQRT><<<g, kBlock, 0, s>>>(x, out, n); break;
    case ABS: k_unary<ABS><<<g, kBlock, 0, s>>>(x, out, n); break;
    case GELU: k_unary<GELU><<<g, kBlock, 0, s>>>(x, out, n); break;
    default: fail("malus: bad unary op %d", op);
  }
  post_launch("unary");
}

void unary_bwd(int op, const float* xy, const float* dout, float* out, size_t n, hipStream_t s) {
  if (!n) return;
  unsigned g = ew_grid(n / 4 + 1);
  switch (op) {
    case B_SIGMOID: k_unary_bwd<B_SIGMOID><<<g, kBlock, 0, s>>>(xy, dout, out, n); break;
    case B_RELU: k_unary_bwd<B_RELU><<<g, kBlock, 0, s>>>(xy, dout, out, n); break;
    case B_TANH: k_unary_bwd<B_TANH><<<g, kBlock, 0, s>>>(xy, dout, out, n); break;
    case B_SQRT: k_unary_bwd<B_SQRT><<<g, kBlock, 0, s>>>(xy, dout, out, n); break;
    case B_ABS: k_unary_bwd<B_ABS><<<g, kBlock, 0, s>>>(xy, dout, out, n); break;
    case B_GELU: k_unary_bwd<B_GELU><<<g, kBlock, 0, s>>>(xy, dout, out, n); break;
    case B_EXP: k_unary_bwd<B_EXP><<<g, kBlock, 0, s>>>(xy, dout, out, n); break;
    case B_LOG: k_unary_bwd<B_LOG><<<g, kBlock, 0, s>>>(xy, dout, out, n); break;
    default: fail("malus: bad unary bwd op %d", op);
  }
  post_launch("unary_bwd");
}

void convert_f32_bf16(const void* x, void* out, size_t n, bool to_bf16, hipStream_t s) {
  if (!n) return;
  if (to_bf16) k_f32_to_bf16<<<ew_grid(n), kBlock, 0, s>>>(static_cast<const float*>(x), static_cast<__bf16*>(out), n);
  else k_bf16_to_f32<<<ew_grid(n), kBlock, 0, s>>>(static_cast<const __bf16*>(x), static_cast<float*>(out), n);
  post_launch("convert");
}

void to_bf16_multi(const Bf16Copy* segs_host, int count, hipStream_t s) {
  for (int base = 0; base < count; base += kCvtMaxSegs) {
    CvtTable t{};
    t.count = count - base < kCvtMaxSegs ? count - base : kCvtMaxSegs;
    size_t chunks = 0;
    for (int i = 0; i < t.count; ++i) {
      t.seg[i] = segs_host[base + i];
      t.first_chunk[i] = (uint32_t)chunks;
      chunks += (t.seg[i].n + kCvtChunk - 1) / kCvtChunk;
    }
    t.first_chunk[t.count] = (uint32_t)chunks;
    if (chunks == 0) continue;
    if (chunks > 0x7fffffffu) fail("malus: bf16 copies: too many elements");
    k_to_bf16_multi<<<(unsigned)chunks, kBlock, 0, s>>>(t);
    post_launch("to_bf16_multi");
  }
}

void to_split3_multi(const Bf16Copy* segs_host, int count, hipStream_t s) {
  for (int base = 0; base < count; base += kCvtMaxSegs) {
    CvtTable t{};
    t.count = count - base < kCvtMaxSegs ? count - base : kCvtMaxSegs;
    size_t chunks = 0;
    for (int i = 0; i < t.count; ++i) {
      t.seg[i] = segs_host[base + i];
      t.first_chunk[i] = (uint32_t)chunks;
      chunks += (t.seg[i].n + kCvtChunk - 1) / kCvtChunk;
    }
    t.first_chunk[t.count] = (uint32_t)chunks;
    if (chunks == 0) continue;
    if (chunks > 0x7fffffffu) fail("malus: split copies: too many elements");
    k_split3_multi<<<(unsigned)chunks, kBlock, 0, s>>>(t);
    post_launch("to_split3_multi");
  }
}

void fill(float* out, float v, size_t n, hipStream_t s) {
  if (!n) return;
  k_fill<<<ew_grid(n / 4 + 1), kBlock, 0, s>>>(out, v, nullptr, n);
  post_launch("fill");
}

void fill_from_device(float* out, const float* v, size_t n, hipStream_t s) {
  if (!n) return;
  k_fill<<<ew_grid(n / 4 + 1), kBlock, 0, s>>>(out, 0.f, v, n);
  post_launch("fill_from_device");
}

void fill_bytes0(void* out, size_t bytes, hipStream_t s) {
  if (!bytes) return;
  k_zero_bytes<<<ew_grid(bytes / 16 + 1), kBlock, 0, s>>>(static_cast<uint8_t*>(out), bytes / 16, bytes);
  post_launch("fill_bytes0");
}

void eq(const float* a, const float* b, float* out, size_t n, hipStream_t s) {
  if (!n) return;
  k_eq<<<ew_grid(n / 4 + 1), kBlock, 0, s>>>(a, b, out, n);
  post_launch("eq");
}

void rsqrt_eps(const float* v, float eps, float* out, size_t n, hipStream_t s) {
  if (!n) return;
  k_rsqrt_eps<<<ew_grid(n), kBlock, 0, s>>>(v, eps, out, n);
  post_launch("rsqrt_eps");
}

void copy(const void* src, void* dst, size_t bytes, hipStream_t s) {
  if (!bytes) return;
  k_copy_bytes<<<ew_grid(bytes / 16 + 1), kBlock, 0, s>>>(static_cast<const uint8_t*>(src), static_cast<uint8_t*>(dst),
                                                          bytes / 16, bytes);
  post_launch("copy");
}

void causal_mask(float* out, size_t t, hipStream_t s) {
  if (!t) return;
  k_causal_mask<<<ew_grid(t * t), kBlock, 0, s>>>(out, (uint32_t)t);
  post_launch("causal_mask");
}

void iota_rows(int32_t* out, size_t rows, size_t t, hipStream_t s) {
  if (!rows || !t) return;
  k_iota_rows<<<ew_grid(rows * t), kBlock, 0, s>>>(out, rows * t, (uint32_t)t);
  post_launch("iota_rows");
}

}  // namespace k
}  // namespace malus
