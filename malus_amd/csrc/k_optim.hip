// Fused "AdamW" step of the reference examples (coupled L2: the decay is
// added to the gradient), examples/nanogpt_modular.ml:97-108.  The reference
// issues ~16 elementwise launches per parameter tensor; this kernel performs
// the same f32 expression tree per element in one pass (reads p, g, m, v;
// writes p', m', v'), so results match the op-by-op sequence bit for bit.
#include <vector>

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

// Multi-tensor form: one launch updates up to kAdamMaxSegs parameter
// tensors.  The segment table travels by value in the kernel arguments (no
// upload).  Block b covers 1024 floats (one float4 per thread) of the
// segment whose chunk range holds b; chunks never straddle segments.  (Per
// launch over the C5 model's 10.77 M parameters: 4096-float chunks 55.0 us,
// 2048 50.8 us, 1024 48.8 us; a linear scan of the segment table instead of
// the binary search cost 1-2 us more.)
// 56 segments: the C5 model's 52 parameter tensors in one launch (one
// ramp-up and drain instead of two), 3.8 KB of kernel arguments.
constexpr int kAdamMaxSegs = 56;
struct AdamTable {
  AdamSeg seg[kAdamMaxSegs];
  uint32_t first_chunk[kAdamMaxSegs + 1];  // prefix sums of the segments' chunk counts
  int count;
};
static_assert(sizeof(AdamTable) + 64 <= 4096, "the segment table travels in the 4 KB of kernel arguments");

// bc (optional): the two bias corrections read from device memory instead of
// the arguments, so a captured step can take each step's values from a
// buffer the host refills before every replay.
__global__ __launch_bounds__(256) void k_adam_l2_multi(const AdamTable t, AdamArgs a, const float* __restrict__ bc) {
  if (bc) {
    a.bc1 = bc[0];
    a.bc2 = bc[1];
  }
  // the segment holding chunk blockIdx.x: the last si with first_chunk[si] <= blockIdx.x
  int lo = 0, hi = t.count - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (t.first_chunk[mid] <= blockIdx.x) lo = mid;
    else hi = mid - 1;
  }
  const int si = lo;
  const AdamSeg& sg = t.seg[si];
  const size_t first = (size_t)(blockIdx.x - t.first_chunk[si]) * kAdamChunk, n = sg.n;
  const size_t end = first + kAdamChunk < n ? first + kAdamChunk : n;
  constexpr int PER = (int)(kAdamChunk / 4 / 256);  // float4 per thread in a whole chunk
  if ((n & 3) == 0 && end - first == kAdamChunk && blockDim.x == 256) {
    // Whole chunk: every load is issued before the first store (the outputs
    // may alias the inputs, in place, so the compiler cannot hoist the next
    // iteration's loads above this one's stores by itself).
    const float4* P4 = reinterpret_cast<const float4*>(sg.p) + first / 4 + threadIdx.x;
    const float4* G4 = reinterpret_cast<const float4*>(sg.g) + first / 4 + threadIdx.x;
    const float4* M4 = reinterpret_cast<const float4*>(sg.m) + first / 4 + threadIdx.x;
    const float4* V4 = reinterpret_cast<const float4*>(sg.v) + first / 4 + threadIdx.x;
    float4 P[PER], G[PER], Mv[PER], V[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      P[j] = P4[256 * j];
      G[j] = G4[256 * j];
      Mv[j] = M4[256 * j];
      V[j] = V4[256 * j];
    }
    float4* Po4 = reinterpret_cast<float4*>(sg.po) + first / 4 + threadIdx.x;
    float4* Mo4 = reinterpret_cast<float4*>(sg.mo) + first / 4 + threadIdx.x;
    float4* Vo4 = reinterpret_cast<float4*>(sg.vo) + first / 4 + threadIdx.x;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      float4 Po, Mo, Vo;
      adam_one(P[j].x, G[j].x, Mv[j].x, V[j].x, a, Po.x, Mo.x, Vo.x);
      adam_one(P[j].y, G[j].y, Mv[j].y, V[j].y, a, Po.y, Mo.y, Vo.y);
      adam_one(P[j].z, G[j].z, Mv[j].z, V[j].z, a, Po.z, Mo.z, Vo.z);
      adam_one(P[j].w, G[j].w, Mv[j].w, V[j].w, a, Po.w, Mo.w, Vo.w);
      Po4[256 * j] = Po;
      Mo4[256 * j] = Mo;
      Vo4[256 * j] = Vo;
    }
  } else if ((n & 3) == 0) {  // float4 path (segment bases are 256-byte aligned)
    for (size_t i = first / 4 + threadIdx.x; i < end / 4; i += blockDim.x) {
      const float4 P = reinterpret_cast<const float4*>(sg.p)[i], G = reinterpret_cast<const float4*>(sg.g)[i];
      const float4 Mv = reinterpret_cast<const float4*>(sg.m)[i], V = reinterpret_cast<const float4*>(sg.v)[i];
      float4 Po, Mo, Vo;
      adam_one(P.x, G.x, Mv.x, V.x, a, Po.x, Mo.x, Vo.x);
      adam_one(P.y, G.y, Mv.y, V.y, a, Po.y, Mo.y, Vo.y);
      adam_one(P.z, G.z, Mv.z, V.z, a, Po.z, Mo.z, Vo.z);
      adam_one(P.w, G.w, Mv.w, V.w, a, Po.w, Mo.w, Vo.w);
      reinterpret_cast<float4*>(sg.po)[i] = Po;
      reinterpret_cast<float4*>(sg.mo)[i] = Mo;
      reinterpret_cast<float4*>(sg.vo)[i] = Vo;
    }
  } else {
    for (size_t i = first + threadIdx.x; i < end; i += blockDim.x)
      adam_one(sg.p[i], sg.g[i], sg.m[i], sg.v[i], a, sg.po[i], sg.mo[i], sg.vo[i]);
  }
}

}  // namespace

void adam_l2_multi(const AdamSeg* segs_host, int count, float lr, float b1, float b2, float omb1, float omb2, float bc1,
                   float bc2, float eps, float wd, hipStream_t s, const float* bc_dev) {
  const AdamArgs a{lr, b1, b2, omb1, omb2, bc1, bc2, eps, wd};
  for (int base = 0; base < count; base += kAdamMaxSegs) {
    AdamTable t{};
    t.count = count - base < kAdamMaxSegs ? count - base : kAdamMaxSegs;
    size_t chunks = 0;
    for (int i = 0; i < t.count; ++i) {
      t.seg[i] = segs_host[base + i];
      t.first_chunk[i] = (uint32_t)chunks;
      chunks += (t.seg[i].n + kAdamChunk - 1) / kAdamChunk;
    }
    t.first_chunk[t.count] = (uint32_t)chunks;
    if (chunks == 0) continue;
    if (chunks > 0x7fffffffu) fail("malus: adam update: too many parameters");
    k_adam_l2_multi<<<(unsigned)chunks, 256, 0, s>>>(t, a, bc_dev);
    MALUS_HIP(hipGetLastError());
  }
}

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
