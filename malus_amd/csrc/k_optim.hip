// Fused "AdamW" step of the reference examples (coupled L2: the decay is
// added to the gradient), examples/nanogpt_modular.ml:97-108.  The reference
// issues ~16 elementwise launches per parameter tensor; this kernel performs
// the same f32 expression tree per element in one pass (reads p, g, m, v;
// writes p', m', v'), so results match the op-by-op sequence bit for bit.
#include "common.h"

namespace malus {
namespace k {
namespace {

struct AdamArgs {
  float lr, b1, b2, omb1, omb2, bc1, bc2, eps, wd;
};

__device__ __forceinline__ void adam_one(float p, float g, float m, float v, const AdamArgs& a, float& po, float& mo,
                                         float& vo) {
  float wdp = p * a.wd;            // opt.wd * ps[i].data      (malus_mul_scalar)
  float gg = g + wdp;              // ps[i].grad + ...          (broadcast add)
  float t1 = m * a.b1;             // opt.beta1 * ms[i]
  float t2 = gg * a.omb1;          // (1.0 - opt.beta1) * g
  float mm = t1 + t2;
  float t3 = v * a.b2;             // opt.beta2 * vs[i]
  float t4 = gg * a.omb2;          // (1.0 - opt.beta2) * g
  float t5 = t4 * gg;              //   ... * g
  float vv = t3 + t5;
  float m_hat = mm / a.bc1;        // ms[i] / bc1               (malus_div_scalar)
  float v_hat = vv / a.bc2;
  float t6 = m_hat * a.lr;         // opt.lr * m_hat
  float t7 = sqrtf(v_hat);
  float t8 = t7 + a.eps;           // sqrt(v_hat) + opt.eps     (malus_add_scalar)
  float t9 = t6 / t8;
  po = p - t9;                     // ps[i].data - ...
  mo = mm;
  vo = vv;
}

__global__ __launch_bounds__(256) void k_adam_l2(const float* __restrict__ p, const float* __restrict__ g,
                                                 const float* __restrict__ m, const float* __restrict__ v,
                                                 float* __restrict__ po, float* __restrict__ mo, float* __restrict__ vo,
                                                 size_t n, AdamArgs a) {
  const size_t n4 = n / 4, stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += stride) {
    float4 P = reinterpret_cast<const float4*>(p)[i], G = reinterpret_cast<const float4*>(g)[i];
    float4 Mv = reinterpret_cast<const float4*>(m)[i], V = reinterpret_cast<const float4*>(v)[i];
    float4 Po, Mo, Vo;
    adam_one(P.x, G.x, Mv.x, V.x, a, Po.x, Mo.x, Vo.x);
    adam_one(P.y, G.y, Mv.y, V.y, a, Po.y, Mo.y, Vo.y);
    adam_one(P.z, G.z, Mv.z, V.z, a, Po.z, Mo.z, Vo.z);
    adam_one(P.w, G.w, Mv.w, V.w, a, Po.w, Mo.w, Vo.w);
    reinterpret_cast<float4*>(po)[i] = Po;
    reinterpret_cast<float4*>(mo)[i] = Mo;
    reinterpret_cast<float4*>(vo)[i] = Vo;
  }
  for (size_t i = n4 * 4 + (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    adam_one(p[i], g[i], m[i], v[i], a, po[i], mo[i], vo[i]);
}

}  // namespace

void adam_l2(const float* p, const float* g, const float* m, const float* v, float* p_out, float* m_out, float* v_out,
             size_t n, float lr, float b1, float b2, float omb1, float omb2, float bc1, float bc2, float eps, float wd,
             hipStream_t s) {
  if (!n) return;
  AdamArgs a{lr, b1, b2, omb1, omb2, bc1, bc2, eps, wd};
  size_t blocks = (n / 4 + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 2048) blocks = 2048;
  k_adam_l2<<<(unsigned)blocks, 256, 0, s>>>(p, g, m, v, p_out, m_out, v_out, n, a);
  MALUS_HIP(hipGetLastError());
}

}  // namespace k
}  // namespace malus
