// Attention scores fused on MFMA: P = softmax(Q K^T * scale + mask) per
// query row, for the head-folded composed attention of
// examples/nanogpt_modular.ml:49-62 (scores = (Q @ Kt) * scale; masked =
// scores + vmask; attn = softmax(masked, axis=2)).
//
// One wave owns 32 query rows and every key of their rows: it computes the
// transposed tile S^T = K Q^T with v_mfma_f32_32x32x2f32, so lane l holds
// query row i = l % 32 and, in its accumulator registers, the keys
//   j = 32 t + 8 (r / 4) + 4 (l / 32) + r % 4     (key tile t, register r).
// The row's max and sum then need one cross-lane step (lanes l and l ^ 32)
// instead of a 32-lane reduction, and S never leaves the registers.
//
// The result is bit-identical to gemm(Q, Kt) followed by
// scale_mask_softmax:
// - each MFMA step pairs the same two k values (k0 + s, k0 + 8 + s of every
//   16-deep slab) in the same order as the GEMM's LDS-staged fragments, and
//   the two products of a step commute;
// - scale, mask add, expf and the division are the same f32 operations;
// - the row sum adds the same 4-element partials in the same tree as the row
//   kernel's wave reduction (xor 32, 16, 8 across key tiles, 4 and 2 across
//   register groups, 1 across the lane pair).
// With a causal mask (-1e9 above the diagonal) the key tiles wholly above a
// wave's rows are not computed: in the composed form their probabilities are
// expf(-1e9 - max) = +0 exactly and their partial sums are +0, which is what
// the kernel stores and adds.
#include "common.h"

namespace malus {
namespace k {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

template <int TT, int HS, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void k_attn_scores_softmax(const float* __restrict__ Q, const float* __restrict__ Kh,
                                                               const float* __restrict__ scale,
                                                               const float* __restrict__ mask, float* __restrict__ P) {
  constexpr int NT = TT / 32;   // key tiles per row (= 32-row query tiles per head)
  constexpr int NKB = HS / 16;  // 16-deep k slabs
  constexpr int LD = HS + 4;    // padded LDS row: 8 consecutive rows of a 128-bit read hit distinct banks
  __shared__ __attribute__((aligned(16))) float Ks[TT * LD];
  const int bh = blockIdx.y;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const size_t head = (size_t)bh * TT * HS;

  // Query tiles are dealt in pairs (p, NT-1-p) so that every workgroup gets
  // the same number of unmasked key tiles under a causal mask.
  const int pair = 2 * blockIdx.x + (wave >> 1);
  const int qt = (wave & 1) ? NT - 1 - pair : pair;
  const bool idle = pair >= (NT + 1) / 2 || ((wave & 1) && qt == pair);  // odd NT: the middle tile has no partner
  const int i0 = 32 * (idle ? 0 : qt);
  const int x = lane & 31, lk = lane >> 5;
  const int live = CAUSAL ? qt + 1 : NT;  // key tiles holding an unmasked key

  // B operand: Q[i0 + x][16 kb + 8 lk + s] for step s of slab kb (loaded
  // while K is staged; an idle wave reads tile 0 and discards it)
  const v4f* qp = reinterpret_cast<const v4f*>(Q + head + (size_t)(i0 + x) * HS + 8 * lk);
  v4f qv[2 * NKB];
#pragma unroll
  for (int e = 0; e < 2 * NKB; ++e) qv[e] = qp[4 * (e >> 1) + (e & 1)];

  // every wave helps stage the head's K in LDS before any wave may leave
  {
    constexpr int N4 = TT * HS / 4, PER = (N4 + 255) / 256;
    const v4f* src = reinterpret_cast<const v4f*>(Kh + head);
    v4f tmp[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int f = threadIdx.x + 256 * u;
      if (f < N4) tmp[u] = src[f];
    }
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int f = threadIdx.x + 256 * u;
      if (f < N4) *reinterpret_cast<v4f*>(Ks + (f / (HS / 4)) * LD + 4 * (f % (HS / 4))) = tmp[u];
    }
  }
  __syncthreads();

  if (idle) return;  // no barrier follows: idle waves leave

  // A operand: K[32 t + x][16 kb + 8 lk + s] from LDS
  v16f acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    acc[t] = v16f{0};
    if (t < live) {
      const float* kr = Ks + (32 * t + x) * LD + 8 * lk;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const v4f a = *reinterpret_cast<const v4f*>(kr + 16 * kb);
        const v4f b = *reinterpret_cast<const v4f*>(kr + 16 * kb + 4);
#pragma unroll
        for (int s = 0; s < 4; ++s) acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], qv[2 * kb][s], acc[t], 0, 0, 0);
#pragma unroll
        for (int s = 0; s < 4; ++s)
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(b[s], qv[2 * kb + 1][s], acc[t], 0, 0, 0);
      }
    }
  }

  // x = S * scale + mask[i][j]; row max.  The causal mask is the one
  // tensor_causal_mask fills: -1e9 where j > i, else 0.
  const int i = i0 + x;
  const float sc = scale[0];
  const v4f* mrow = reinterpret_cast<const v4f*>(mask + (size_t)i * TT);
  float m = -INFINITY;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if (t < live) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        v4f mk;
        if (CAUSAL) {  // only the diagonal tile (t == qt) mixes masked and unmasked keys
#pragma unroll
          for (int c = 0; c < 4; ++c) mk[c] = t == qt && 32 * t + 8 * g + 4 * lk + c > i ? -1e9f : 0.0f;
        } else {
          mk = mrow[8 * t + 2 * g + lk];
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float ss = acc[t][4 * g + c] * sc;
          const float xv = ss + mk[c];
          acc[t][4 * g + c] = xv;
          m = fmaxf(m, xv);
        }
      }
    }
  }
  m = fmaxf(m, __shfl_xor(m, 32, 64));

  // probabilities and the per-group partial sums v[t][g] (4 keys each)
  float v[NT][4];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float s = 0.0f;
      if (t < live) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float ex = expf(acc[t][4 * g + c] - m);
          acc[t][4 * g + c] = ex;
          s += ex;
        }
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[t][4 * g + c] = 0.0f;
      }
      v[t][g] = s;
    }
  }
  // the row kernel's xor tree over 4-key groups gi = 8 t + 2 g + lk:
  // bits 5..3 of gi are t's, bits 2..1 are g's, bit 0 is the lane pair
#pragma unroll
  for (int tb = NT / 2; tb >= 1; tb >>= 1)
#pragma unroll
    for (int t = 0; t < tb; ++t)
#pragma unroll
      for (int g = 0; g < 4; ++g) v[t][g] = v[t][g] + v[t + tb][g];
  float s = 0.0f;
  {
    const float d0 = v[0][0] + v[0][2], d1 = v[0][1] + v[0][3];
    s = d0 + d1;
  }
  s = s + __shfl_xor(s, 32, 64);

  v4f* prow = reinterpret_cast<v4f*>(P + ((size_t)bh * TT + i) * TT);
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      v4f o = v4f{0.0f, 0.0f, 0.0f, 0.0f};  // +0 / s = +0 for the skipped tiles
      if (t < live) {
#pragma unroll
        for (int c = 0; c < 4; ++c) o[c] = acc[t][4 * g + c] / s;
      }
      prow[8 * t + 2 * g + lk] = o;
    }
}

template <int TT, int HS>
void launch(const float* Q, const float* K, const float* scale, const float* mask, float* P, int bh, bool causal,
            hipStream_t s) {
  const dim3 grid((TT / 32 + 3) / 4, (unsigned)bh);  // two query-tile pairs per workgroup
  if (causal) k_attn_scores_softmax<TT, HS, true><<<grid, 256, 0, s>>>(Q, K, scale, mask, P);
  else k_attn_scores_softmax<TT, HS, false><<<grid, 256, 0, s>>>(Q, K, scale, mask, P);
}

// Backward of the scores: dS = softmax_bwd(P, dP) * scale with dP = dO V^T,
// for tape.rs:1150-1161 (dx = s * (dout - sum(dout * s))) followed by the
// scale multiply's VJP (dout * scale).  The wave layout is the forward
// kernel's (lane = query row, registers = keys), so dP^T = V dO^T runs on
// MFMA with V staged in LDS, the row sum is one cross-lane step, and dP never
// reaches memory.  Bit-identical to gemm(dO, V^T), softmax_bwd and the
// scalar multiply: the same MFMA k pairing, per-group products summed from 0
// in key order, the row kernel's xor tree, and the same f32 operations.
// Causal: key tiles above a wave's rows hold P = 0, so their dS is 0 (the
// composed ops give +-0 there) and neither dP nor P is read for them.
// dO of head bh, row i, column d sits at dO + (bh / H) * T * ldo + (bh % H) * HS + i * ldo + d
// (ldo = H * HS: the [B*T, C] attention output read in place).
template <int TT, int HS, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void k_attn_scores_bwd(const float* __restrict__ dO, int ldo, int H,
                                                           const float* __restrict__ V, const float* __restrict__ P,
                                                           const float* __restrict__ scale, float* __restrict__ dS) {
  constexpr int NT = TT / 32;
  constexpr int NKB = HS / 16;
  constexpr int LD = HS + 4;
  __shared__ __attribute__((aligned(16))) float Vs[TT * LD];
  const int bh = blockIdx.y;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const size_t head = (size_t)bh * TT * HS;

  const int pair = 2 * blockIdx.x + (wave >> 1);
  const int qt = (wave & 1) ? NT - 1 - pair : pair;
  const bool idle = pair >= (NT + 1) / 2 || ((wave & 1) && qt == pair);
  const int i0 = 32 * (idle ? 0 : qt);
  const int x = lane & 31, lk = lane >> 5;
  const int live = CAUSAL ? qt + 1 : NT;

  // B operand: dO[i0 + x][16 kb + 8 lk + s]
  const v4f* op = reinterpret_cast<const v4f*>(dO + (size_t)(bh / H) * TT * ldo + (size_t)(bh % H) * HS +
                                               (size_t)(i0 + x) * ldo + 8 * lk);
  v4f ov[2 * NKB];
#pragma unroll
  for (int e = 0; e < 2 * NKB; ++e) ov[e] = op[4 * (e >> 1) + (e & 1)];
  {
    constexpr int N4 = TT * HS / 4, PER = (N4 + 255) / 256;
    const v4f* src = reinterpret_cast<const v4f*>(V + head);
    v4f tmp[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int f = threadIdx.x + 256 * u;
      if (f < N4) tmp[u] = src[f];
    }
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int f = threadIdx.x + 256 * u;
      if (f < N4) *reinterpret_cast<v4f*>(Vs + (f / (HS / 4)) * LD + 4 * (f % (HS / 4))) = tmp[u];
    }
  }
  __syncthreads();
  if (idle) return;  // no barrier follows

  v16f acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    acc[t] = v16f{0};
    if (t < live) {
      const float* vr = Vs + (32 * t + x) * LD + 8 * lk;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const v4f a = *reinterpret_cast<const v4f*>(vr + 16 * kb);
        const v4f b = *reinterpret_cast<const v4f*>(vr + 16 * kb + 4);
#pragma unroll
        for (int s = 0; s < 4; ++s) acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], ov[2 * kb][s], acc[t], 0, 0, 0);
#pragma unroll
        for (int s = 0; s < 4; ++s)
          acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(b[s], ov[2 * kb + 1][s], acc[t], 0, 0, 0);
      }
    }
  }

  // per-group sums of dP * P, then the row kernel's tree
  const int i = i0 + x;
  const v4f* prow = reinterpret_cast<const v4f*>(P + ((size_t)bh * TT + i) * TT);
  float v[NT][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float sum = 0.0f;
      if (t < live) {
        const v4f pv = prow[8 * t + 2 * g + lk];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float pr = acc[t][4 * g + c] * pv[c];
          sum += pr;
        }
      }
      v[t][g] = sum;
    }
#pragma unroll
  for (int tb = NT / 2; tb >= 1; tb >>= 1)
#pragma unroll
    for (int t = 0; t < tb; ++t)
#pragma unroll
      for (int g = 0; g < 4; ++g) v[t][g] = v[t][g] + v[t + tb][g];
  float d = 0.0f;
  {
    const float d0 = v[0][0] + v[0][2], d1 = v[0][1] + v[0][3];
    d = d0 + d1;
  }
  d = d + __shfl_xor(d, 32, 64);

  const float sc = scale[0];
  v4f* srow = reinterpret_cast<v4f*>(dS + ((size_t)bh * TT + i) * TT);
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      v4f o = v4f{0.0f, 0.0f, 0.0f, 0.0f};
      if (t < live) {
        const v4f pv = prow[8 * t + 2 * g + lk];  // second read of the row (cache): dP stays in registers
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float diff = acc[t][4 * g + c] - d;
          const float dx = pv[c] * diff;
          o[c] = dx * sc;
        }
      }
      srow[8 * t + 2 * g + lk] = o;
    }
}

template <int TT, int HS>
void launch_bwd(const float* dO, int ldo, int H, const float* V, const float* P, const float* scale, float* dS, int bh,
                bool causal, hipStream_t s) {
  const dim3 grid((TT / 32 + 3) / 4, (unsigned)bh);
  if (causal) k_attn_scores_bwd<TT, HS, true><<<grid, 256, 0, s>>>(dO, ldo, H, V, P, scale, dS);
  else k_attn_scores_bwd<TT, HS, false><<<grid, 256, 0, s>>>(dO, ldo, H, V, P, scale, dS);
}

}  // namespace

bool attn_scores_supported(size_t bh, size_t t, size_t hs) {
  if (bh == 0 || bh > 65535) return false;
  return (t == 256 && hs == 64) || (t == 128 && hs == 64) || (t == 64 && hs == 32) || (t == 64 && hs == 64);
}

bool attn_scores_softmax(const float* Q, const float* K, const float* scale, const float* mask, float* P, size_t bh,
                         size_t t, size_t hs, bool causal, hipStream_t s) {
  if (!attn_scores_supported(bh, t, hs)) return false;
  const auto aligned = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (!aligned(Q) || !aligned(K) || !aligned(mask) || !aligned(P) || (!causal && !mask)) return false;
  const int b = (int)bh;
  if (t == 256 && hs == 64) launch<256, 64>(Q, K, scale, mask, P, b, causal, s);
  else if (t == 128 && hs == 64) launch<128, 64>(Q, K, scale, mask, P, b, causal, s);
  else if (t == 64 && hs == 32) launch<64, 32>(Q, K, scale, mask, P, b, causal, s);
  else if (t == 64 && hs == 64) launch<64, 64>(Q, K, scale, mask, P, b, causal, s);
  else return false;
  MALUS_HIP(hipGetLastError());
  return true;
}

bool attn_scores_bwd(const float* dO, size_t ldo, size_t heads, const float* V, const float* P, const float* scale,
                     float* dS, size_t bh, size_t t, size_t hs, bool causal, hipStream_t s) {
  if (!attn_scores_supported(bh, t, hs) || heads == 0 || bh % heads || ldo < hs * heads) return false;
  const auto aligned = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (!aligned(dO) || !aligned(V) || !aligned(P) || !aligned(dS) || ldo % 4) return false;
  const int b = (int)bh, l = (int)ldo, H = (int)heads;
  if (t == 256 && hs == 64) launch_bwd<256, 64>(dO, l, H, V, P, scale, dS, b, causal, s);
  else if (t == 128 && hs == 64) launch_bwd<128, 64>(dO, l, H, V, P, scale, dS, b, causal, s);
  else if (t == 64 && hs == 32) launch_bwd<64, 32>(dO, l, H, V, P, scale, dS, b, causal, s);
  else if (t == 64 && hs == 64) launch_bwd<64, 64>(dO, l, H, V, P, scale, dS, b, causal, s);
  else return false;
  MALUS_HIP(hipGetLastError());
  return true;
}

}  // namespace k
}  // namespace malus
