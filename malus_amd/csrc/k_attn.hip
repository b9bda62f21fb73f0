// Attention fused on MFMA: P = softmax(Q K^T * scale + mask) per query row
// and att = P @ V, for the head-folded composed attention of
// examples/nanogpt_modular.ml:49-62 (scores = (Q @ Kt) * scale; masked =
// scores + vmask; attn = softmax(masked, axis=2); attn @ V).
//
// One wave owns 32 query rows and every key of their rows: it computes the
// transposed tile S^T = K Q^T with v_mfma_f32_32x32x2f32, so lane l holds
// query row i = l % 32 and the keys of its row sit in its accumulator
// registers.  The row's max and sum then need one cross-lane step (lanes l
// and l ^ 32) instead of a 32-lane reduction, and S never leaves the
// registers.  The K rows are fed to the MFMA with bits 2 and 3 of the row
// index swapped (key_row), so lane half lk holds, in register r = 4 g + c of
// key tile t, the key
//   32 t + 16 (g >> 1) + 8 lk + 4 (g & 1) + c.
// Registers 8 h .. 8 h + 7 of tile t are then keys 32 t + 16 h + 8 lk + s,
// s = 0 .. 7: the A operand of MFMA step s of the 16-deep k slab 2 t + h in
// a product with P on the left.  So P @ V (forward) and dS @ K (backward)
// run from the registers, with V or K staged in LDS.
//
// The results are bit-identical to gemm(Q, Kt), scale_mask_softmax and
// gemm(P, V):
// - each MFMA step pairs the same two k values (k0 + s, k0 + 8 + s of every
//   16-deep slab) in the same order as the GEMM's LDS-staged fragments, and
//   the two products of a step commute;
// - scale, mask add, expf and the division are the same f32 operations;
// - the row sum adds the same 4-element partials in the same tree as the row
//   kernel's wave reduction (row_tree).
// With a causal mask (-1e9 above the diagonal) the key tiles wholly above a
// wave's rows are not computed: in the composed form their probabilities are
// expf(-1e9 - max) = +0 exactly and their partial sums are +0, which is what
// the kernel stores and adds, and their products with V add exact zeros.
#include "common.h"
#include "k_split.h"

namespace malus {
namespace k {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

// The key tile row an MFMA A-operand lane x loads: bits 2 and 3 swapped.
__device__ __forceinline__ int key_row(int x) { return x ^ ((((x >> 2) ^ (x >> 3)) & 1) * 12); }
// The 4-key group (key / 4) in register group g of lane half lk, tile t.
__device__ __forceinline__ int key_group(int t, int g, int lk) { return 8 * t + 4 * (g >> 1) + 2 * lk + (g & 1); }

// The row kernel's xor tree over the row's 4-key group partials, indexed by
// gi = key_group(t, g, lk): bits 5..3 of gi are t's (xor 32, 16, 8), bit 2
// is g >> 1 (xor 4), bit 1 the lane half (xor 2: lanes l and l ^ 32), bit 0
// is g & 1 (xor 1).  Both lanes of a pair return the sum.
template <int NT>
__device__ __forceinline__ float row_tree(float (&v)[NT][4]) {
#pragma unroll
  for (int tb = NT / 2; tb >= 1; tb >>= 1)
#pragma unroll
    for (int t = 0; t < tb; ++t)
#pragma unroll
      for (int g = 0; g < 4; ++g) v[t][g] = v[t][g] + v[t + tb][g];
  float d0 = v[0][0] + v[0][2], d1 = v[0][1] + v[0][3];
  d0 = d0 + __shfl_xor(d0, 32, 64);
  d1 = d1 + __shfl_xor(d1, 32, 64);
  return d0 + d1;
}

// Stage one head's [TT, HS] matrix in LDS with padded rows (LD = HS + 4:
// 8 consecutive rows of a 128-bit read hit distinct banks).
template <int TT, int HS>
__device__ __forceinline__ void stage_head(const float* __restrict__ src_head, float* S) {
  constexpr int LD = HS + 4, N4 = TT * HS / 4, PER = (N4 + 255) / 256;
  const v4f* src = reinterpret_cast<const v4f*>(src_head);
  v4f tmp[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int f = threadIdx.x + 256 * u;
    if (f < N4) tmp[u] = src[f];
  }
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int f = threadIdx.x + 256 * u;
    if (f < N4) *reinterpret_cast<v4f*>(S + (f / (HS / 4)) * LD + 4 * (f % (HS / 4))) = tmp[u];
  }
}

// out[off(n, r)] = (D[off(n, r)] +) o[n][r] for a wave's [32, 32 NN] result:
// every addend is loaded before the first add, so the loads overlap.
template <int NN, typename Off>
__device__ __forceinline__ void store_tile(const v16f (&o)[NN], float* __restrict__ out, const float* __restrict__ D,
                                           Off off) {
  if (D) {
    float d[NN][16];
#pragma unroll
    for (int n = 0; n < NN; ++n)
#pragma unroll
      for (int r = 0; r < 16; ++r) d[n][r] = D[off(n, r)];
#pragma unroll
    for (int n = 0; n < NN; ++n)
#pragma unroll
      for (int r = 0; r < 16; ++r) out[off(n, r)] = d[n][r] + o[n][r];
  } else {
#pragma unroll
    for (int n = 0; n < NN; ++n)
#pragma unroll
      for (int r = 0; r < 16; ++r) out[off(n, r)] = o[n][r];
  }
}

// out[i0 + i][d] (+ D) = sum over the live key tiles of A[i][key] M[key][d],
// with A in the key-tile registers of the layout above and M staged in LDS
// (padded rows).  The slabs run in key order, as the GEMM's do.  out/D of
// row i, column d sit at i * ld + d from the head's base.
template <int NT, int HS, bool X3>
__device__ __forceinline__ void product_from_registers(const v16f (&a)[NT], int live, const float* Ms, int i0,
                                                       float* __restrict__ out, const float* __restrict__ D, int ld) {
  constexpr int LD = HS + 4, NN = HS / 32;
  const int lane = threadIdx.x & 63, x = lane & 31, lk = lane >> 5;
  v16f o[1][NN];
#pragma unroll
  for (int n = 0; n < NN; ++n) o[0][n] = v16f{0};
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if (t < live) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if constexpr (X3) {  // slab 2 t + h: keys 32 t + 16 h + 8 lk + s
          float af[8], bf[NN][8];
#pragma unroll
          for (int s = 0; s < 8; ++s) {
            af[s] = a[t][8 * h + s];
            const float* mr = Ms + (32 * t + 16 * h + 8 * lk + s) * LD + x;
#pragma unroll
            for (int n = 0; n < NN; ++n) bf[n][s] = mr[32 * n];
          }
          Split3 sa[1] = {split3(af)}, sb[NN];
#pragma unroll
          for (int n = 0; n < NN; ++n) sb[n] = split3(bf[n]);
          x3_slab<false, 1, NN>(sa, sb, o);
        } else {
#pragma unroll
          for (int s = 0; s < 8; ++s) {
            const float* mr = Ms + (32 * t + 16 * h + 8 * lk + s) * LD + x;
#pragma unroll
            for (int n = 0; n < NN; ++n)
              o[0][n] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t][8 * h + s], mr[32 * n], o[0][n], 0, 0, 0);
          }
        }
      }
    }
  }
  __builtin_amdgcn_s_setprio(0);
  store_tile<NN>(o[0], out, D, [&](int n, int r) { return (size_t)(i0 + 8 * (r >> 2) + 4 * lk + (r & 3)) * ld + 32 * n + x; });
}

// Stage one head's [TT, HS] rows that sit ld floats apart (the [B*T, C]
// layout read in place) in LDS with padded rows, as stage_head does.
template <int TT, int HS>
__device__ __forceinline__ void stage_rows(const float* __restrict__ src_head, int ld, float* S) {
  constexpr int LD = HS + 4, N4 = TT * HS / 4, PER = (N4 + 255) / 256;
  v4f tmp[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int f = threadIdx.x + 256 * u;
    if (f < N4) tmp[u] = *reinterpret_cast<const v4f*>(src_head + (size_t)(f / (HS / 4)) * ld + 4 * (f % (HS / 4)));
  }
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int f = threadIdx.x + 256 * u;
    if (f < N4) *reinterpret_cast<v4f*>(S + (f / (HS / 4)) * LD + 4 * (f % (HS / 4))) = tmp[u];
  }
}

// out[32 j + i][d] (+ D) = sum over queries q of A[q][32 j + i] M[q][d]: the
// product A^T M for key tile j, A a head's [TT, TT] matrix in global memory
// (P or dS) and M [TT, HS] staged in LDS (padded rows).  The queries run in
// 16-deep slabs in ascending order and MFMA step s of a slab pairs queries
// k0 + s (lane half 0) and k0 + 8 + s (lane half 1), exactly as the GEMM's
// fragments of a transposed A operand do, so the values are the GEMM's.
// Causal: the slabs before query 32 j are skipped; there A holds +0 or -0
// (P = 0 above the diagonal), and the GEMM either skips them too or adds
// those zero products to a +0 accumulator.  A's slab pairs are loaded two
// pairs ahead of their MFMAs.  out/D rows are HS floats apart.
// SWAP (split products): the composed ops form this product with the
// operands in the other roles (dK: the VJP of Q @ Kt with respect to Kt is
// Q^T @ dS, then permuted), so the piece products run in that GEMM's order.
template <int TT, int HS, bool CAUSAL, bool X3, bool SWAP>
__device__ __forceinline__ void transposed_product(const float* __restrict__ Ah, int j, const float* Ms,
                                                   float* __restrict__ out, const float* __restrict__ D) {
  constexpr int LD = HS + 4, NN = HS / 32, NSL = TT / 16;
  const int lane = threadIdx.x & 63, x = lane & 31, lk = lane >> 5;
  const int s0 = CAUSAL ? 2 * j : 0;  // a key tile spans two slabs, so the slab count is even
  const float* ap = Ah + 32 * j + x + (size_t)(8 * lk) * TT;
  auto load = [&](int sl, float (&r)[16]) {
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int s = 0; s < 8; ++s) r[8 * u + s] = ap[(size_t)(16 * (sl + u) + s) * TT];
  };
  v16f o[1][NN];
#pragma unroll
  for (int n = 0; n < NN; ++n) o[0][n] = v16f{0};
  constexpr int PD = 2;  // slab pairs loaded ahead of their MFMAs (one ahead measured 1.5 % slower)
  float a[PD + 1][16];
#pragma unroll
  for (int d = 0; d < PD; ++d) {
#pragma unroll
    for (int e = 0; e < 16; ++e) a[d][e] = 0.0f;
    if (s0 + 2 * d < NSL) load(s0 + 2 * d, a[d]);
  }
  for (int sl = s0; sl < NSL; sl += 2) {
#pragma unroll
    for (int e = 0; e < 16; ++e) a[PD][e] = 0.0f;
    if (sl + 2 * PD < NSL) load(sl + 2 * PD, a[PD]);
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      if constexpr (X3) {  // slab sl + u: queries 16 (sl + u) + 8 lk + s
        float af[8], bf[NN][8];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          af[s] = a[0][8 * u + s];
          const float* mr = Ms + (16 * (sl + u) + 8 * lk + s) * LD + x;
#pragma unroll
          for (int n = 0; n < NN; ++n) bf[n][s] = mr[32 * n];
        }
        Split3 sa[1] = {split3(af)}, sb[NN];
#pragma unroll
        for (int n = 0; n < NN; ++n) sb[n] = split3(bf[n]);
        x3_slab<SWAP, 1, NN>(sa, sb, o);
      } else {
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const float* mr = Ms + (16 * (sl + u) + 8 * lk + s) * LD + x;
#pragma unroll
          for (int n = 0; n < NN; ++n)
            o[0][n] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[0][8 * u + s], mr[32 * n], o[0][n], 0, 0, 0);
        }
      }
    }
    __builtin_amdgcn_s_setprio(0);
#pragma unroll
    for (int d = 0; d < PD; ++d)
#pragma unroll
      for (int e = 0; e < 16; ++e) a[d][e] = a[d + 1][e];
  }
  store_tile<NN>(o[0], out, D, [&](int n, int r) { return (size_t)(32 * j + 8 * (r >> 2) + 4 * lk + (r & 3)) * HS + 32 * n + x; });
}

// Query tiles are dealt to the waves in pairs (p, NT-1-p): wave w runs both
// tiles of pair w, one after the other, so every wave has NT + 1 key tiles
// of unmasked work under a causal mask and the workgroup (one head) is
// balanced across its SIMDs.  NT <= 8: at most four pairs per head.
template <int NT>
__device__ __forceinline__ int pair_tile(int w, int which) {
  return which ? NT - 1 - w : w;
}

// One wave's query tile qt (rows 32 qt ..): S^T = K Q^T from K staged in LDS
// (rows in key_row order), scale, mask, the row softmax, and the store of the
// P rows.  Leaves P in acc (zeros in the skipped key tiles).
template <int TT, int HS, bool CAUSAL, bool X3>
__device__ __forceinline__ void softmax_tile(const float* __restrict__ Qh, const float* Ks, const float* __restrict__ scale,
                                             const float* __restrict__ mask, float* __restrict__ Ph, int qt,
                                             v16f (&acc)[TT / 32], bool full) {
  constexpr int NT = TT / 32;   // key tiles per row (= 32-row query tiles per head)
  constexpr int NKB = HS / 16;  // 16-deep k slabs
  constexpr int LD = HS + 4;
  const int lane = threadIdx.x & 63, x = lane & 31, lk = lane >> 5;
  const int i0 = 32 * qt, i = i0 + x;
  const int live = CAUSAL ? qt + 1 : NT;  // key tiles holding an unmasked key

  // B operand: Q[i0 + x][16 kb + 8 lk + s] for step s of slab kb
  const v4f* qp = reinterpret_cast<const v4f*>(Qh + (size_t)i * HS + 8 * lk);
  v4f qv[2 * NKB];
#pragma unroll
  for (int e = 0; e < 2 * NKB; ++e) qv[e] = qp[4 * (e >> 1) + (e & 1)];

  // A operand: K[32 t + key_row(x)][16 kb + 8 lk + s] from LDS
  __builtin_amdgcn_s_setprio(1);  // MFMA issue ahead of the CU's other waves
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    acc[t] = v16f{0};
    if (t < live) {
      const float* kr = Ks + (32 * t + key_row(x)) * LD + 8 * lk;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const v4f a = *reinterpret_cast<const v4f*>(kr + 16 * kb);
        const v4f b = *reinterpret_cast<const v4f*>(kr + 16 * kb + 4);
        if constexpr (X3) {  // S^T = K Q^T: the composed GEMM's operands swapped
          const float af[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
          const float bf[8] = {qv[2 * kb][0], qv[2 * kb][1], qv[2 * kb][2], qv[2 * kb][3],
                               qv[2 * kb + 1][0], qv[2 * kb + 1][1], qv[2 * kb + 1][2], qv[2 * kb + 1][3]};
          acc[t] = x3_one<true>(split3(af), split3(bf), acc[t]);
        } else {
#pragma unroll
          for (int s = 0; s < 4; ++s) acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], qv[2 * kb][s], acc[t], 0, 0, 0);
#pragma unroll
          for (int s = 0; s < 4; ++s)
            acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(b[s], qv[2 * kb + 1][s], acc[t], 0, 0, 0);
        }
      }
    }
  }

  __builtin_amdgcn_s_setprio(0);

  // x = S * scale + mask[i][j]; row max.  The causal mask is the one
  // tensor_causal_mask fills: -1e9 where j > i, else 0.
  const float sc = scale[0];
  const v4f* mrow = reinterpret_cast<const v4f*>(mask + (size_t)i * TT);
  float m = -INFINITY;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    if (t < live) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int gi = key_group(t, g, lk);
        v4f mk;
        if (CAUSAL) {  // only the diagonal tile (t == qt) mixes masked and unmasked keys
#pragma unroll
          for (int c = 0; c < 4; ++c) mk[c] = t == qt && 4 * gi + c > i ? -1e9f : 0.0f;
        } else {
          mk = mrow[gi];
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
  const float s = row_tree<NT>(v);

  v4f* prow = reinterpret_cast<v4f*>(Ph + (size_t)i * TT);
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      v4f o = v4f{0.0f, 0.0f, 0.0f, 0.0f};  // +0 / s = +0 for the skipped tiles
      if (t < live) {
#pragma unroll
        for (int c = 0; c < 4; ++c) o[c] = acc[t][4 * g + c] = acc[t][4 * g + c] / s;
      }
      if (t < live || full) prow[key_group(t, g, lk)] = o;
    }
}

// Reload a wave's [32, TT] rows (P or dS of query tile qt, stored by
// softmax_tile / dscores_tile) into the key-tile register layout; the
// skipped key tiles are zero.
template <int TT>
__device__ __forceinline__ void load_tile(const float* __restrict__ Xh, int qt, int live, v16f (&acc)[TT / 32]) {
  constexpr int NT = TT / 32;
  const int lane = threadIdx.x & 63, x = lane & 31, lk = lane >> 5;
  const v4f* row = reinterpret_cast<const v4f*>(Xh + (size_t)(32 * qt + x) * TT);
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const v4f q = t < live ? row[key_group(t, g, lk)] : v4f{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[t][4 * g + c] = q[c];
    }
}

// PV: also att = P @ V, written at O + (bh / H) * TT * ldo + (bh % H) * HS
// + i * ldo + d (ldo = H * HS: the [B*T, C] layout the output projection
// reads; ldo = HS, H = 1: dense heads).  One workgroup per head; wave w
// runs query tiles w and NT-1-w: both score tiles while K is staged (the
// first one's P goes to memory, the second stays in registers), then, with V
// staged where K was, P @ V for the second tile from the registers and for
// the first from its reloaded rows.
template <int TT, int HS, bool CAUSAL, bool PV, bool X3>
__global__ __launch_bounds__(256, 2) void k_attn_fwd(const float* __restrict__ Q, const float* __restrict__ Kh,
                                                    const float* __restrict__ V, const float* __restrict__ scale,
                                                    const float* __restrict__ mask, float* __restrict__ P,
                                                    float* __restrict__ O, int ldo, int H, bool full) {
  constexpr int NT = TT / 32;
  constexpr int LD = HS + 4;
  static_assert(NT % 2 == 0 && NT <= 8, "one pair of query tiles per wave");
  __shared__ __attribute__((aligned(16))) float S[TT * LD];  // K, then V
  const int bh = blockIdx.y;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const size_t head = (size_t)bh * TT * HS;
  const bool active = wave < NT / 2;
  const int qa = pair_tile<NT>(wave, 0), qb = pair_tile<NT>(wave, 1);
  float* Ph = P + (size_t)bh * TT * TT;

  stage_head<TT, HS>(Kh + head, S);
  __syncthreads();
  v16f acc[NT];
  if (active) {
    softmax_tile<TT, HS, CAUSAL, X3>(Q + head, S, scale, mask, Ph, qa, acc, full);
    softmax_tile<TT, HS, CAUSAL, X3>(Q + head, S, scale, mask, Ph, qb, acc, full);
  }
  if constexpr (PV) {
    __syncthreads();  // every wave is done with K
    stage_head<TT, HS>(V + head, S);
    __syncthreads();
    if (active) {
      float* Oh = O + (size_t)(bh / H) * TT * ldo + (size_t)(bh % H) * HS;
      product_from_registers<NT, HS, X3>(acc, CAUSAL ? qb + 1 : NT, S, 32 * qb, Oh, nullptr, ldo);
      load_tile<TT>(Ph, qa, CAUSAL ? qa + 1 : NT, acc);
      product_from_registers<NT, HS, X3>(acc, CAUSAL ? qa + 1 : NT, S, 32 * qa, Oh, nullptr, ldo);
    }
  }
}

template <int TT, int HS, bool X3>
void launch_prec(const float* Q, const float* K, const float* V, const float* scale, const float* mask, float* P,
                 float* O, int ldo, int H, int bh, bool causal, bool full, hipStream_t s) {
  const dim3 grid(1, (unsigned)bh);  // one workgroup per head
  if (O) {
    if (causal) k_attn_fwd<TT, HS, true, true, X3><<<grid, 256, 0, s>>>(Q, K, V, scale, mask, P, O, ldo, H, full);
    else k_attn_fwd<TT, HS, false, true, X3><<<grid, 256, 0, s>>>(Q, K, V, scale, mask, P, O, ldo, H, true);
  } else {
    if (causal) k_attn_fwd<TT, HS, true, false, X3><<<grid, 256, 0, s>>>(Q, K, V, scale, mask, P, O, ldo, H, full);
    else k_attn_fwd<TT, HS, false, false, X3><<<grid, 256, 0, s>>>(Q, K, V, scale, mask, P, O, ldo, H, true);
  }
}

// The products run as the GEMMs run theirs (gemm_f32_split), so the fused
// kernels keep the composed ops' bits.
template <int TT, int HS>
void launch(const float* Q, const float* K, const float* V, const float* scale, const float* mask, float* P, float* O,
            int ldo, int H, int bh, bool causal, bool full, hipStream_t s) {
  if (gemm_f32_split()) launch_prec<TT, HS, true>(Q, K, V, scale, mask, P, O, ldo, H, bh, causal, full, s);
  else launch_prec<TT, HS, false>(Q, K, V, scale, mask, P, O, ldo, H, bh, causal, full, s);
}

// Zero the 32 x 32 tiles of P [bh, TT, TT] wholly above the diagonal: one
// 256-thread workgroup per (head, query tile), float4 stores.
__global__ __launch_bounds__(256) void k_attn_zero_upper(float* __restrict__ P, int TT) {
  const int NT = TT / 32, qt = (int)blockIdx.x % NT;
  const size_t bh = blockIdx.x / NT;
  const int first = 32 * (qt + 1), n4 = (TT - first) / 4;  // float4s per row right of the diagonal tile
  float* rows = P + (bh * TT + 32 * (size_t)qt) * TT + first;
  for (int f = threadIdx.x; f < 32 * n4; f += 256)
    reinterpret_cast<v4f*>(rows + (size_t)(f / n4) * TT)[f % n4] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
}

// One wave's query tile qt of the scores backward: dP^T = V dO^T from V
// staged in LDS, dS = P * (dP - sum(dP * P)) * scale, and the store of the dS
// rows.  Leaves dS in acc.
template <int TT, int HS, bool CAUSAL, bool X3>
__device__ __forceinline__ void dscores_tile(const float* __restrict__ dOh, int ldo, const float* Vs,
                                             const float* __restrict__ Ph, const float* __restrict__ scale,
                                             float* __restrict__ dSh, int qt, v16f (&acc)[TT / 32], bool full) {
  constexpr int NT = TT / 32;
  constexpr int NKB = HS / 16;
  constexpr int LD = HS + 4;
  const int lane = threadIdx.x & 63, x = lane & 31, lk = lane >> 5;
  const int i0 = 32 * qt, i = i0 + x;
  const int live = CAUSAL ? qt + 1 : NT;

  // B operand: dO[i0 + x][16 kb + 8 lk + s]
  const v4f* op = reinterpret_cast<const v4f*>(dOh + (size_t)i * ldo + 8 * lk);
  v4f ov[2 * NKB];
#pragma unroll
  for (int e = 0; e < 2 * NKB; ++e) ov[e] = op[4 * (e >> 1) + (e & 1)];
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    acc[t] = v16f{0};
    if (t < live) {
      const float* vr = Vs + (32 * t + key_row(x)) * LD + 8 * lk;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        const v4f a = *reinterpret_cast<const v4f*>(vr + 16 * kb);
        const v4f b = *reinterpret_cast<const v4f*>(vr + 16 * kb + 4);
        if constexpr (X3) {  // dP^T = V dO^T: the composed GEMM's operands swapped
          const float af[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
          const float bf[8] = {ov[2 * kb][0], ov[2 * kb][1], ov[2 * kb][2], ov[2 * kb][3],
                               ov[2 * kb + 1][0], ov[2 * kb + 1][1], ov[2 * kb + 1][2], ov[2 * kb + 1][3]};
          acc[t] = x3_one<true>(split3(af), split3(bf), acc[t]);
        } else {
#pragma unroll
          for (int s = 0; s < 4; ++s) acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], ov[2 * kb][s], acc[t], 0, 0, 0);
#pragma unroll
          for (int s = 0; s < 4; ++s)
            acc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(b[s], ov[2 * kb + 1][s], acc[t], 0, 0, 0);
        }
      }
    }
  }

  __builtin_amdgcn_s_setprio(0);

  // per-group sums of dP * P, then the row kernel's tree
  const v4f* prow = reinterpret_cast<const v4f*>(Ph + (size_t)i * TT);
  float v[NT][4];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float sum = 0.0f;
      if (t < live) {
        const v4f pv = prow[key_group(t, g, lk)];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float pr = acc[t][4 * g + c] * pv[c];
          sum += pr;
        }
      }
      v[t][g] = sum;
    }
  const float d = row_tree<NT>(v);

  const float sc = scale[0];
  v4f* srow = reinterpret_cast<v4f*>(dSh + (size_t)i * TT);
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      v4f o = v4f{0.0f, 0.0f, 0.0f, 0.0f};
      if (t < live) {
        const v4f pv = prow[key_group(t, g, lk)];  // second read of the row (cache): dP stays in registers
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float diff = acc[t][4 * g + c] - d;
          const float dx = pv[c] * diff;
          o[c] = acc[t][4 * g + c] = dx * sc;
        }
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[t][4 * g + c] = 0.0f;
      }
      if (t < live || full) srow[key_group(t, g, lk)] = o;
    }
}

// Backward of the scores: dS = softmax_bwd(P, dP) * scale with dP = dO V^T,
// for tape.rs:1150-1161 (dx = s * (dout - sum(dout * s))) followed by the
// scale multiply's VJP (dout * scale); DQ: also dQ = dS @ K (+ Dq), the
// scores product's VJP for Q.  The wave layout is the forward kernel's
// (lane = query row, registers = keys in the key_row order, one pair of
// query tiles per wave), so dP^T = V dO^T runs on MFMA with V staged in LDS,
// the row sum is one cross-lane step, dP never reaches memory, and dS feeds
// dS @ K from the registers (the pair's second tile) or from its reloaded
// rows (the first) with K staged in LDS after V.  Bit-identical to
// gemm(dO, V^T), softmax_bwd, the scalar multiply and gemm(dS, K): the same
// MFMA k pairing, per-group products summed from 0 in key order, the row
// kernel's xor tree, and the same f32 operations.
// Causal: key tiles above a wave's rows hold P = 0, so their dS is 0 (the
// composed ops give +-0 there) and neither dP nor P is read for them.
// dO of head bh, row i, column d sits at dO + (bh / H) * T * ldo + (bh % H) * HS + i * ldo + d
// (ldo = H * HS: the [B*T, C] attention output read in place).
// KV: then also dV = P^T dO (dO staged in LDS) and dK = dS^T Q (Q staged),
// each wave taking the key tiles of its pair (the same balance as the query
// tiles: under a causal mask key tile j meets the NT - j query tiles from j
// on).  The dS rows other waves stored are read back after a barrier.
template <int TT, int HS, bool CAUSAL, bool DQ, bool KV, bool X3>
__global__ __launch_bounds__(256, 2) void k_attn_bwd(const float* __restrict__ dO, int ldo, int H,
                                                    const float* __restrict__ V, const float* __restrict__ P,
                                                    const float* __restrict__ scale, float* __restrict__ dS,
                                                    const float* __restrict__ Kh, float* __restrict__ dQ,
                                                    const float* __restrict__ Dq, AttnKV kv, bool full) {
  constexpr int NT = TT / 32;
  constexpr int LD = HS + 4;
  static_assert(NT % 2 == 0 && NT <= 8, "one pair of query tiles per wave");
  __shared__ __attribute__((aligned(16))) float S[TT * LD];  // V, then K
  const int bh = blockIdx.y;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const size_t head = (size_t)bh * TT * HS;
  const bool active = wave < NT / 2;
  const int qa = pair_tile<NT>(wave, 0), qb = pair_tile<NT>(wave, 1);
  const float* dOh = dO + (size_t)(bh / H) * TT * ldo + (size_t)(bh % H) * HS;
  const float* Ph = P + (size_t)bh * TT * TT;
  float* dSh = dS + (size_t)bh * TT * TT;

  stage_head<TT, HS>(V + head, S);
  __syncthreads();
  v16f acc[NT];
  if (active) {
    dscores_tile<TT, HS, CAUSAL, X3>(dOh, ldo, S, Ph, scale, dSh, qa, acc, full);
    dscores_tile<TT, HS, CAUSAL, X3>(dOh, ldo, S, Ph, scale, dSh, qb, acc, full);
  }
  if constexpr (DQ) {
    __syncthreads();  // every wave is done with V
    stage_head<TT, HS>(Kh + head, S);
    __syncthreads();
    if (active) {
      const float* Dh = Dq ? Dq + head : nullptr;
      product_from_registers<NT, HS, X3>(acc, CAUSAL ? qb + 1 : NT, S, 32 * qb, dQ + head, Dh, HS);
      load_tile<TT>(dSh, qa, CAUSAL ? qa + 1 : NT, acc);
      product_from_registers<NT, HS, X3>(acc, CAUSAL ? qa + 1 : NT, S, 32 * qa, dQ + head, Dh, HS);
    }
  }
  if constexpr (KV) {
    __syncthreads();  // every wave is done with K and has stored its dS rows
    stage_rows<TT, HS>(dOh, ldo, S);
    __syncthreads();
    if (active) {
      const float* Dv = kv.Dv ? kv.Dv + head : nullptr;
      transposed_product<TT, HS, CAUSAL, X3, false>(Ph, qa, S, kv.dV + head, Dv);  // P^T @ dO
      transposed_product<TT, HS, CAUSAL, X3, false>(Ph, qb, S, kv.dV + head, Dv);
    }
    __syncthreads();  // every wave is done with dO
    stage_head<TT, HS>(kv.Q + head, S);
    __syncthreads();
    if (active) {
      const float* Dk = kv.Dk ? kv.Dk + head : nullptr;
      transposed_product<TT, HS, CAUSAL, X3, true>(dSh, qa, S, kv.dK + head, Dk);  // (Q^T @ dS)^T
      transposed_product<TT, HS, CAUSAL, X3, true>(dSh, qb, S, kv.dK + head, Dk);
    }
  }
}

template <int TT, int HS, bool X3>
void launch_bwd_prec(const float* dO, int ldo, int H, const float* V, const float* P, const float* scale, float* dS,
                     const float* K, float* dQ, const float* Dq, int bh, bool causal, const AttnKV* kv, bool full,
                     hipStream_t s) {
  const dim3 grid(1, (unsigned)bh);  // one workgroup per head
  const AttnKV a = kv ? *kv : AttnKV{};
  if (kv) {
    if (causal)
      k_attn_bwd<TT, HS, true, true, true, X3><<<grid, 256, 0, s>>>(dO, ldo, H, V, P, scale, dS, K, dQ, Dq, a, full);
    else
      k_attn_bwd<TT, HS, false, true, true, X3><<<grid, 256, 0, s>>>(dO, ldo, H, V, P, scale, dS, K, dQ, Dq, a, true);
  } else if (dQ) {
    if (causal)
      k_attn_bwd<TT, HS, true, true, false, X3><<<grid, 256, 0, s>>>(dO, ldo, H, V, P, scale, dS, K, dQ, Dq, a, full);
    else
      k_attn_bwd<TT, HS, false, true, false, X3><<<grid, 256, 0, s>>>(dO, ldo, H, V, P, scale, dS, K, dQ, Dq, a, true);
  } else {
    if (causal)
      k_attn_bwd<TT, HS, true, false, false, X3><<<grid, 256, 0, s>>>(dO, ldo, H, V, P, scale, dS, K, dQ, Dq, a, full);
    else
      k_attn_bwd<TT, HS, false, false, false, X3><<<grid, 256, 0, s>>>(dO, ldo, H, V, P, scale, dS, K, dQ, Dq, a, true);
  }
}

template <int TT, int HS>
void launch_bwd(const float* dO, int ldo, int H, const float* V, const float* P, const float* scale, float* dS,
                const float* K, float* dQ, const float* Dq, int bh, bool causal, const AttnKV* kv, bool full,
                hipStream_t s) {
  if (gemm_f32_split())
    launch_bwd_prec<TT, HS, true>(dO, ldo, H, V, P, scale, dS, K, dQ, Dq, bh, causal, kv, full, s);
  else
    launch_bwd_prec<TT, HS, false>(dO, ldo, H, V, P, scale, dS, K, dQ, Dq, bh, causal, kv, full, s);
}

}  // namespace

bool attn_scores_supported(size_t bh, size_t t, size_t hs) {
  if (bh == 0 || bh > 65535) return false;
  return (t == 256 && hs == 64) || (t == 128 && hs == 64) || (t == 64 && hs == 32) || (t == 64 && hs == 64);
}

bool attn_fwd(const float* Q, const float* K, const float* V, const float* scale, const float* mask, float* P, float* O,
              size_t ldo, size_t heads, size_t bh, size_t t, size_t hs, bool causal, hipStream_t s, bool full) {
  if (!attn_scores_supported(bh, t, hs)) return false;
  const auto aligned = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (!aligned(Q) || !aligned(K) || !aligned(mask) || !aligned(P) || (!causal && !mask)) return false;
  if (O && (!V || !aligned(V) || !aligned(O) || ldo % 4 || heads == 0 || bh % heads || ldo < hs * heads)) return false;
  const int b = (int)bh, l = (int)ldo, H = (int)heads;
  if (t == 256 && hs == 64) launch<256, 64>(Q, K, V, scale, mask, P, O, l, H, b, causal, full, s);
  else if (t == 128 && hs == 64) launch<128, 64>(Q, K, V, scale, mask, P, O, l, H, b, causal, full, s);
  else if (t == 64 && hs == 32) launch<64, 32>(Q, K, V, scale, mask, P, O, l, H, b, causal, full, s);
  else if (t == 64 && hs == 64) launch<64, 64>(Q, K, V, scale, mask, P, O, l, H, b, causal, full, s);
  else return false;
  MALUS_HIP(hipGetLastError());
  return true;
}

void attn_zero_upper_tiles(float* P, size_t bh, size_t t, hipStream_t s) {
  if (!bh || t < 64 || t % 32 || bh * (t / 32) > 0x7fffffffu) return;
  k_attn_zero_upper<<<(unsigned)(bh * (t / 32)), 256, 0, s>>>(P, (int)t);
  MALUS_HIP(hipGetLastError());
}

bool attn_scores_softmax(const float* Q, const float* K, const float* scale, const float* mask, float* P, size_t bh,
                         size_t t, size_t hs, bool causal, hipStream_t s) {
  return attn_fwd(Q, K, nullptr, scale, mask, P, nullptr, 0, 0, bh, t, hs, causal, s);
}

bool attn_bwd(const float* dO, size_t ldo, size_t heads, const float* V, const float* P, const float* scale, float* dS,
              const float* K, float* dQ, const float* Dq, size_t bh, size_t t, size_t hs, bool causal, hipStream_t s,
              const AttnKV* kv, bool full) {
  if (!attn_scores_supported(bh, t, hs) || heads == 0 || bh % heads || ldo < hs * heads) return false;
  const auto aligned = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  if (!aligned(dO) || !aligned(V) || !aligned(P) || !aligned(dS) || ldo % 4) return false;
  if (dQ && (!K || !aligned(K) || !aligned(dQ) || (Dq && !aligned(Dq)))) return false;
  if (kv && (!dQ || !kv->Q || !kv->dK || !kv->dV || !aligned(kv->Q) || !aligned(kv->dK) || !aligned(kv->dV) ||
             (kv->Dk && !aligned(kv->Dk)) || (kv->Dv && !aligned(kv->Dv))))
    return false;
  const int b = (int)bh, l = (int)ldo, H = (int)heads;
  if (t == 256 && hs == 64) launch_bwd<256, 64>(dO, l, H, V, P, scale, dS, K, dQ, Dq, b, causal, kv, full, s);
  else if (t == 128 && hs == 64) launch_bwd<128, 64>(dO, l, H, V, P, scale, dS, K, dQ, Dq, b, causal, kv, full, s);
  else if (t == 64 && hs == 32) launch_bwd<64, 32>(dO, l, H, V, P, scale, dS, K, dQ, Dq, b, causal, kv, full, s);
  else if (t == 64 && hs == 64) launch_bwd<64, 64>(dO, l, H, V, P, scale, dS, K, dQ, Dq, b, causal, kv, full, s);
  else return false;
  MALUS_HIP(hipGetLastError());
  return true;
}

bool attn_scores_bwd(const float* dO, size_t ldo, size_t heads, const float* V, const float* P, const float* scale,
                     float* dS, size_t bh, size_t t, size_t hs, bool causal, hipStream_t s) {
  return attn_bwd(dO, ldo, heads, V, P, scale, dS, nullptr, nullptr, nullptr, bh, t, hs, causal, s);
}

}  // namespace k
}  // namespace malus
