// GELU and its VJP as device functions, shared by the elementwise kernels and
// the GEMM epilogues that fuse them, so both evaluate the same expressions
// (tensor_gelu, metal.rs:1535-1549; VJP tape.rs:1187-1199; the CPU fallback's
// order ((c1 x) x) x and its constants).  Built with -ffp-contract=off.
#pragma once

#include <hip/hip_runtime.h>

namespace malus {
namespace k {

// tanh for GELU's inner argument: 1 - 2 / (1 + 2^(2 y log2 e)) with the
// hardware exp2 and reciprocal (each within 1 ulp).  Its absolute error is
// at most 3 ulp(1) for every y (no cancellation issue: GELU adds the result
// to 1, so only absolute error matters), and e -> inf / 0 give exactly
// +1 / -1.  It replaces the library tanhf's ~35 instructions with ~5, which
// keeps the GELU kernels memory-bound.
__device__ __forceinline__ float gelu_tanh(float y) {
  const float e = __builtin_amdgcn_exp2f(y * 2.8853900817779268f);  // 2 / ln 2
  const float r = __builtin_amdgcn_rcpf(1.0f + e);
  return __builtin_fmaf(-2.0f, r, 1.0f);
}

__device__ __forceinline__ float gelu_fwd(float x) {
  const float C0 = 0.7978845608f, C1 = 0.044715f;
  float inner = C0 * (x + C1 * x * x * x);
  return 0.5f * x * (1.0f + gelu_tanh(inner));
}

// d * gelu'(v)
__device__ __forceinline__ float gelu_bwd(float v, float d) {
  const float C0 = 0.7978845608f, C1 = 0.044715f;
  float g = C0 * (v + C1 * v * v * v);
  float t = gelu_tanh(g);
  float gp = C0 * (1.0f + 3.0f * C1 * v * v);
  float deriv = 0.5f * (1.0f + t) + 0.5f * v * (1.0f - t * t) * gp;
  return d * deriv;
}

}  // namespace k
}  // namespace malus
