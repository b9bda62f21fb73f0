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

// Multi-tensor form: one launch updates every parameter tensor.  Block b
// takes chunk[b] = (segment, first float) and covers 4096 floats of that
// segment (1024 float4, four per thread); chunks never straddle segments.
__global__ __launch_bounds__(256) void k_adam_l2_multi(const AdamSeg* __restrict__ segs, const uint2* __restrict__ chunks,
                                                       AdamArgs a) {
  const uint2 ch = chunks[blockIdx.x];
  const AdamSeg sg = segs[ch.x];
  const size_t first = ch.y, n = sg.n;
  const size_t end = first + kAdamChunk < n ? first + kAdamChunk : n;
  if ((n & 3) == 0) {  // float4 path (segment bases are 256-byte aligned)
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
                   float bc2, float eps, float wd, hipStream_t s) {
  std::vector<uint2> chunks;
  for (int i = 0; i < count; ++i)
    for (size_t f = 0; f < segs_host[i].n; f += kAdamChunk) chunks.push_back(make_uint2((unsigned)i, (unsigned)f));
  if (chunks.empty()) return;
  if (chunks.size() > 0x7fffffffu) fail("malus: adam update: too many parameters");
  // segment table and chunk table ride one device buffer
  const size_t seg_bytes = (size_t)count * sizeof(AdamSeg), chunk_bytes = chunks.size() * sizeof(uint2);
  const size_t off = (seg_bytes + 255) / 256 * 256;
  size_t bucket;
  char* dev = static_cast<char*>(pool_alloc(off + chunk_bytes, &bucket));
  upload(dev, segs_host, seg_bytes);
  upload(dev + off, chunks.data(), chunk_bytes);
  AdamArgs a{lr, b1, b2, omb1, omb2, bc1, bc2, eps, wd};
  k_adam_l2_multi<<<(unsigned)chunks.size(), 256, 0, s>>>(reinterpret_cast<const AdamSeg*>(dev),
                                                          reinterpret_cast<const uint2*>(dev + off), a);
  MALUS_HIP(hipGetLastError());
  pool_free(dev, bucket);  // stream order keeps it alive until the kernel has read it
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
