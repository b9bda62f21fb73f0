// Flash attention: causal (or unmasked) softmax(Q K^T * scale) @ V with an
// online softmax (Dao et al.), the post-composed attention that
// docs/adr/0029-composed-attention.md:23-33 reserves: the [B*H, T, T]
// scores and probabilities are never written; the forward keeps one f32 per
// query row (lse = max + log(sum)), and the backward recomputes P from it.
// T is any multiple of 32 (no softmax-row cap); head sizes 32 and 64.
//
// Work split: one wave per (head, 32-row tile); the grid runs the longest
// tiles first (under a causal mask query tile q meets q + 1 key tiles, key
// tile k meets NT - k query tiles), so the scheduler balances the CUs with
// 64-thread workgroups.  Of each product one operand is held in registers
// for the whole pass (Q, dO of the query tile; K, V of the key tile) and the
// other streams from L2; a streamed tile needed in a transposed orientation
// (V in the forward, K in dQ, Q and dO in the f32 dK/dV) is staged in LDS.
//
// MFMA layout (v_mfma_f32_32x32x2f32; under autocast one
// v_mfma_f32_32x32x16_bf16 per 16-deep slab; with split f32 products (X3,
// k_split.h) six of them per slab on the operands' exact bf16 pieces, the
// operand a pass holds in registers split once per pass): lane l = x + 32 lk supplies
// row / column x of its operand; in each 16-deep slab lane half lk supplies
// the 8 consecutive k values 8 lk .. 8 lk + 7.  The accumulator of lane l
// holds column x and rows 8 (r >> 2) + 4 lk + (r & 3), r = 0..15.  A row
// operand loaded through perm_row (bits 2 and 3 of the row swapped) leaves
// register r holding row perm_index(r, lk) = 16 (r >> 3) + 8 lk + (r & 7):
// registers 8 h .. 8 h + 7 are then a slab's k values for the next product,
// so P and dS feed the P V, dS K, dO^T P and Q^T dS products from registers.
//
// Backward: dS = P * (dP - D) * scale with D = rowsum(dO * O) (equal to the
// composed softmax VJP's rowsum(dP * P) in exact arithmetic); dQ from a
// query-centric pass (S^T, dP^T, dQ += dS K), dK and dV from a key-centric
// pass (S, dP, dV^T += dO^T P, dK^T += Q^T dS).  Each gradient element is
// written by one wave: no atomics, and the results are deterministic.
#include "common.h"
#include "k_split.h"

namespace malus {
namespace k {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ int perm_row(int x) { return x ^ ((((x >> 2) ^ (x >> 3)) & 1) * 12); }
__device__ __forceinline__ int perm_index(int r, int lk) { return 16 * (r >> 3) + 8 * lk + (r & 7); }

// One 16-deep slab: acc += A B over the 8 k values of each lane half.
template <bool BF, bool X3 = false>
__device__ __forceinline__ v16f slab(const float (&a)[8], const float (&b)[8], v16f c) {
  if constexpr (X3) {
    return x3_one<false>(split3(a), split3(b), c);
  } else if constexpr (BF) {
    bf16x8 x, y;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x[e] = (__bf16)a[e];
      y[e] = (__bf16)b[e];
    }
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, y, c, 0, 0, 0);
  } else {
#pragma unroll
    for (int s = 0; s < 8; ++s) c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], b[s], c, 0, 0, 0);
    return c;
  }
}

// 8 consecutive floats (16-byte aligned)
__device__ __forceinline__ void load8(const float* __restrict__ p, float (&v)[8]) {
  const v4f a = *reinterpret_cast<const v4f*>(p), b = *reinterpret_cast<const v4f*>(p + 4);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[e] = a[e];
    v[4 + e] = b[e];
  }
}

// Q, K, V and their gradients in the model's storage type: f32, or bf16
// under the autocast storage policy (S16; element offsets either way).  A
// bf16 value widens to f32 exactly, and the bf16 MFMA rounds it back to
// itself, so the products see the same operands as from an f32 copy of the
// rounded values.
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
template <bool S16>
__device__ __forceinline__ void ld8(const float* __restrict__ base, size_t i, float (&v)[8]) {
  if constexpr (S16) {
    const bf16x8 h = *reinterpret_cast<const bf16x8*>(reinterpret_cast<const __bf16*>(base) + i);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (float)h[e];
  } else {
    load8(base + i, v);
  }
}
template <bool S16>
__device__ __forceinline__ v4f ld4(const float* __restrict__ base, size_t i) {
  if constexpr (S16) {
    const bf16x4 h = *reinterpret_cast<const bf16x4*>(reinterpret_cast<const __bf16*>(base) + i);
    return v4f{(float)h[0], (float)h[1], (float)h[2], (float)h[3]};
  } else {
    return *reinterpret_cast<const v4f*>(base + i);
  }
}
template <bool S16>
__device__ __forceinline__ float ld1(const float* __restrict__ base, size_t i) {
  if constexpr (S16) return (float)reinterpret_cast<const __bf16*>(base)[i];
  else return base[i];
}
template <bool S16>
__device__ __forceinline__ void st4(float* __restrict__ base, size_t i, v4f w) {
  if constexpr (S16)
    *reinterpret_cast<bf16x4*>(reinterpret_cast<__bf16*>(base) + i) = bf16x4{(__bf16)w[0], (__bf16)w[1], (__bf16)w[2], (__bf16)w[3]};
  else *reinterpret_cast<v4f*>(base + i) = w;
}
template <bool S16>
__device__ __forceinline__ void st1(float* __restrict__ base, size_t i, float w) {
  if constexpr (S16) reinterpret_cast<__bf16*>(base)[i] = (__bf16)w;
  else base[i] = w;
}

// A head's row `row` of a [B*T, H*HS] tensor (O, dO) or of [B*H, T, HS].
__device__ __forceinline__ const float* head_row(const float* base, int bh, int H, int T, int ld, int hs, int row) {
  return base + (size_t)(bh / H) * T * ld + (size_t)(bh % H) * hs + (size_t)row * ld;
}

// Orders one wave's LDS traffic between its lanes: the stores before it are
// visible to every lane's loads after it, and every lane's loads before it
// are done before the stores after it.  Wavefront-scope fences around the
// wave barrier keep the compiler from moving LDS accesses across it; the
// hardware already runs one wave's LDS operations in order, so in these
// one-wave workgroups it costs no instruction.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Forward: query tile qt of head bh.  O^T = V^T P^T keeps the output with
// lane = query, so the online rescale is a per-lane factor.
template <int HS, bool CAUSAL, bool BF, bool S16 = false, bool X3 = false>
__global__ __launch_bounds__(64, 2) void k_flash_fwd(const float* __restrict__ Q, const float* __restrict__ K,
                                                  const float* __restrict__ V, const float* __restrict__ scale,
                                                  float* __restrict__ O, int ldo, int H, float* __restrict__ lse, int T,
                                                  int BH) {
  static_assert(BF || !S16, "bf16 storage runs on the bf16 MFMA");
  constexpr int NKB = HS / 16, NN = HS / 32;
  const int NT = T / 32;
  const int qt = NT - 1 - (int)(blockIdx.x / BH), bh = (int)(blockIdx.x % BH);
  const int lane = threadIdx.x, x = lane & 31, lk = lane >> 5;
  const size_t head = (size_t)bh * T * HS;
  const int i0 = 32 * qt;
  const float sc = scale[0];

  float qb[NKB][8];  // B of S^T = K Q^T: Q[i0 + x][16 kb + 8 lk + e]
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) ld8<S16>(Q, head + (size_t)(i0 + x) * HS + 16 * kb + 8 * lk, qb[kb]);
  float ka[NKB][8];  // A of S^T: K[32 j + perm_row(x)][16 kb + 8 lk + e]
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) ld8<S16>(K, head + (size_t)perm_row(x) * HS + 16 * kb + 8 * lk, ka[kb]);
  Split3 qs[X3 ? NKB : 1];
  if constexpr (X3)
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) qs[kb] = split3(qb[kb]);

  v16f o[NN];
#pragma unroll
  for (int n = 0; n < NN; ++n) o[n] = v16f{0};
  float m = -INFINITY, l = 0.0f;
  const int last = CAUSAL ? qt : NT - 1;
  // Key tile j of V goes through LDS (rows padded to HS + 4 floats): one
  // 16-byte global load per 4 floats, and V^T's columns read back from LDS
  // (1-5 % faster than a 4-byte load per column element).
  constexpr int LD = HS + 4, Q4 = HS / 4, PER = 32 * Q4 / 64;
  __shared__ __attribute__((aligned(16))) float Vs[32 * LD];
  for (int j = 0; j <= last; ++j) {
    float va[NN][2][8];  // A of O^T = V^T P^T: V[32 j + 16 h + 8 lk + e][32 n + x]
    {
      v4f vn[PER];
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        const int f = lane + 64 * u;
        vn[u] = ld4<S16>(V, head + (size_t)(32 * j + f / Q4) * HS + 4 * (f % Q4));
      }
      wave_lds_sync();  // the last tile's reads of Vs are done
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        const int f = lane + 64 * u;
        *reinterpret_cast<v4f*>(Vs + (f / Q4) * LD + 4 * (f % Q4)) = vn[u];
      }
      wave_lds_sync();  // this tile's stores are visible to every lane
#pragma unroll
      for (int n = 0; n < NN; ++n)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int e = 0; e < 8; ++e) va[n][h][e] = Vs[(16 * h + 8 * lk + e) * LD + 32 * n + x];
    }
    v16f st = v16f{0};
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      if constexpr (X3) st = x3_one<false>(split3(ka[kb]), qs[kb], st);
      else st = slab<BF>(ka[kb], qb[kb], st);
    }
    if (j < last) {
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
        ld8<S16>(K, head + (size_t)(32 * (j + 1) + perm_row(x)) * HS + 16 * kb + 8 * lk, ka[kb]);
    }
    // lane = query i0 + x, register r = key 32 j + perm_index(r, lk)
    float mt = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float v = st[r] * sc;
      if (CAUSAL && j == qt && perm_index(r, lk) > x) v = -INFINITY;
      st[r] = v;
      mt = fmaxf(mt, v);
    }
    mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
    const float mn = fmaxf(m, mt);
    const float alpha = expf(m - mn);  // 0 on the first tile (m = -inf)
    float ls = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float p = expf(st[r] - mn);
      st[r] = p;
      ls += p;
    }
    ls += __shfl_xor(ls, 32, 64);
    l = l * alpha + ls;
    m = mn;
#pragma unroll
    for (int n = 0; n < NN; ++n) o[n] *= alpha;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float pb[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) pb[e] = st[8 * h + e];
      if constexpr (X3) {
        const Split3 ps = split3(pb);
#pragma unroll
        for (int n = 0; n < NN; ++n) o[n] = x3_one<false>(split3(va[n][h]), ps, o[n]);
      } else {
#pragma unroll
        for (int n = 0; n < NN; ++n) o[n] = slab<BF>(va[n][h], pb, o[n]);
      }
    }
  }
  // O[i0 + x][32 n + 8 g + 4 lk + c] = o[n][4 g + c] / l
  float* orow = O + (size_t)(bh / H) * T * ldo + (size_t)(bh % H) * HS + (size_t)(i0 + x) * ldo;
#pragma unroll
  for (int n = 0; n < NN; ++n)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      v4f w;
#pragma unroll
      for (int c = 0; c < 4; ++c) w[c] = o[n][4 * g + c] / l;
      *reinterpret_cast<v4f*>(orow + 32 * n + 8 * g + 4 * lk) = w;
    }
  if (lk == 0) lse[(size_t)bh * T + i0 + x] = m + logf(l);
}

// Backward, query-centric: dQ (+ Dq) of query tile qt, and D = rowsum(dO*O)
// of its rows into dsum for the key-centric pass.  W waves per workgroup:
// W = 1, one query tile; W = 4, query tiles 4 g .. 4 g + 3 of one head, one
// per wave, sharing each staged key tile (each thread stages a quarter of it,
// so tile j + 1's loads are issued before tile j's products without the
// registers of a whole tile per wave).  Each wave's products are the same
// either way.
template <int HS, bool CAUSAL, bool BF, bool S16 = false, bool X3 = false, int W = 1>
__global__ __launch_bounds__(64 * W, 2) void k_flash_bwd_dq(const float* __restrict__ Q, const float* __restrict__ K,
                                                     const float* __restrict__ V, const float* __restrict__ O,
                                                     const float* __restrict__ dO, int ldo, int H,
                                                     const float* __restrict__ lse, const float* __restrict__ scale,
                                                     float* __restrict__ dQ, const float* __restrict__ Dq,
                                                     float* __restrict__ dsum, int T, int BH) {
  constexpr int NKB = HS / 16, NN = HS / 32;
  const int NT = T / 32;
  const int lane = threadIdx.x % 64, x = lane & 31, lk = lane >> 5, wave = threadIdx.x / 64;
  // W = 1: the longest tiles first; W = 4: the groups of four tiles, longest first
  const int qt = W == 1 ? NT - 1 - (int)(blockIdx.x / BH) : W * (NT / W - 1 - (int)(blockIdx.x / BH)) + wave;
  const int bh = (int)(blockIdx.x % BH);
  const size_t head = (size_t)bh * T * HS;
  const int i0 = 32 * qt, i = i0 + x;
  const float sc = scale[0];

  float qb[NKB][8], ob[NKB][8];  // B of S^T = K Q^T and of dP^T = V dO^T
  const float* dorow = head_row(dO, bh, H, T, ldo, HS, i);
  const float* orow = head_row(O, bh, H, T, ldo, HS, i);
  float d = 0.0f;
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    ld8<S16>(Q, head + (size_t)i * HS + 16 * kb + 8 * lk, qb[kb]);
    load8(dorow + 16 * kb + 8 * lk, ob[kb]);
    float ov[8];
    load8(orow + 16 * kb + 8 * lk, ov);
#pragma unroll
    for (int e = 0; e < 8; ++e) d += ob[kb][e] * ov[e];
  }
  d += __shfl_xor(d, 32, 64);
  if (lk == 0) dsum[(size_t)bh * T + i] = d;
  Split3 qs[X3 ? NKB : 1], os[X3 ? NKB : 1];
  if constexpr (X3)
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      qs[kb] = split3(qb[kb]);
      os[kb] = split3(ob[kb]);
    }
  const float L = lse[(size_t)bh * T + i];

  v16f dq[NN];
#pragma unroll
  for (int n = 0; n < NN; ++n) dq[n] = v16f{0};
  const int last = CAUSAL ? qt : NT - 1;
  // the workgroup's key tiles: its longest wave's
  const int jmax = W == 1 ? last : (CAUSAL ? W * (qt / W) + W - 1 : NT - 1);
  // Key tile j of K and V goes through LDS (rows padded to HS + 4 floats):
  // one 16-byte global load per 4 floats, and both of K's orientations (the
  // rows for S^T, the columns for dQ = dS K) read back from LDS.  (With one
  // wave per workgroup, fetching tile j + 1 into registers during tile j
  // measured no faster and spilled.)
  constexpr int LD = HS + 4, Q4 = HS / 4, PER = 32 * Q4 / (64 * W);
  __shared__ __attribute__((aligned(16))) float Ks[32 * LD], Vs[32 * LD];
  v4f kn[PER], vn[PER];
  auto fetch = [&](int j) {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int f = threadIdx.x + 64 * W * u;
      kn[u] = ld4<S16>(K, head + (size_t)(32 * j + f / Q4) * HS + 4 * (f % Q4));
      vn[u] = ld4<S16>(V, head + (size_t)(32 * j + f / Q4) * HS + 4 * (f % Q4));
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int f = threadIdx.x + 64 * W * u;
      *reinterpret_cast<v4f*>(Ks + (f / Q4) * LD + 4 * (f % Q4)) = kn[u];
      *reinterpret_cast<v4f*>(Vs + (f / Q4) * LD + 4 * (f % Q4)) = vn[u];
    }
  };
  if (W > 1) fetch(0);
  for (int j = 0; j <= jmax; ++j) {
    if (W == 1) {
      fetch(j);
      wave_lds_sync();  // the last tile's reads of Ks and Vs are done
      stage();
      wave_lds_sync();  // this tile's stores are visible to every lane
    } else {
      __syncthreads();  // every wave's reads of the last tile are done
      stage();
      __syncthreads();  // this tile is visible to every wave
      if (j < jmax) fetch(j + 1);  // in flight during this tile's products
      if (j > last) continue;      // past this wave's diagonal: the barriers only
    }
    float ka[NKB][8], vr[NKB][8];  // A of S^T and dP^T: rows perm_row(x) of K_j, V_j
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      load8(Ks + perm_row(x) * LD + 16 * kb + 8 * lk, ka[kb]);
      load8(Vs + perm_row(x) * LD + 16 * kb + 8 * lk, vr[kb]);
    }
    v16f st = v16f{0}, dp = v16f{0};
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      if constexpr (X3) {
        st = x3_one<false>(split3(ka[kb]), qs[kb], st);
        dp = x3_one<false>(split3(vr[kb]), os[kb], dp);
      } else {
        st = slab<BF>(ka[kb], qb[kb], st);
        dp = slab<BF>(vr[kb], ob[kb], dp);
      }
    }
    float kc[NN][2][8];  // B of dQ = dS K: K[32 j + 16 h + 8 lk + e][32 n + x]
#pragma unroll
    for (int n = 0; n < NN; ++n)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) kc[n][h][e] = Ks[(16 * h + 8 * lk + e) * LD + 32 * n + x];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const bool masked = CAUSAL && j == qt && perm_index(r, lk) > x;
      const float p = masked ? 0.0f : expf(st[r] * sc - L);
      const float diff = dp[r] - d;
      const float dx = p * diff;
      st[r] = dx * sc;
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float ab[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) ab[e] = st[8 * h + e];
      if constexpr (X3) {
        const Split3 as = split3(ab);
#pragma unroll
        for (int n = 0; n < NN; ++n) dq[n] = x3_one<false>(as, split3(kc[n][h]), dq[n]);
      } else {
#pragma unroll
        for (int n = 0; n < NN; ++n) dq[n] = slab<BF>(ab, kc[n][h], dq[n]);
      }
    }
  }
  // dQ[i0 + 8 (r >> 2) + 4 lk + (r & 3)][32 n + x] (+ Dq: every addend loaded
  // before the first add; f32 storage only)
  auto off = [&](int n, int r) { return head + (size_t)(i0 + 8 * (r >> 2) + 4 * lk + (r & 3)) * HS + 32 * n + x; };
  if (!S16 && Dq) {
    float a[NN][16];
#pragma unroll
    for (int n = 0; n < NN; ++n)
#pragma unroll
      for (int r = 0; r < 16; ++r) a[n][r] = Dq[off(n, r)];
#pragma unroll
    for (int n = 0; n < NN; ++n)
#pragma unroll
      for (int r = 0; r < 16; ++r) dQ[off(n, r)] = a[n][r] + dq[n][r];
  } else {
#pragma unroll
    for (int n = 0; n < NN; ++n)
#pragma unroll
      for (int r = 0; r < 16; ++r) st1<S16>(dQ, off(n, r), dq[n][r]);
  }
}

// Backward, key-centric: dK (+ Dk) and dV (+ Dv) of key tile kt.  W waves
// per workgroup as in the dQ pass: W = 4 runs key tiles 4 g .. 4 g + 3 of one
// head, one per wave, sharing each staged query tile (f32 staging only).
template <int HS, bool CAUSAL, bool BF, bool S16 = false, bool X3 = false, int W = 1>
__global__ __launch_bounds__(64 * W, 2) void k_flash_bwd_dkv(const float* __restrict__ Q, const float* __restrict__ K,
                                                      const float* __restrict__ V, const float* __restrict__ dO, int ldo,
                                                      int H, const float* __restrict__ lse,
                                                      const float* __restrict__ dsum, const float* __restrict__ scale,
                                                      float* __restrict__ dK, const float* __restrict__ Dk,
                                                      float* __restrict__ dV, const float* __restrict__ Dv, int T,
                                                      int BH) {
  constexpr int NKB = HS / 16, NN = HS / 32;
  const int NT = T / 32;
  const int lane = threadIdx.x % 64, x = lane & 31, lk = lane >> 5, wave = threadIdx.x / 64;
  const int kt = W * (int)(blockIdx.x / BH) + wave, bh = (int)(blockIdx.x % BH);
  const size_t head = (size_t)bh * T * HS;
  const int j0 = 32 * kt, key = j0 + x;
  const float sc = scale[0];
  const float* lseh = lse + (size_t)bh * T;
  const float* dsh = dsum + (size_t)bh * T;

  float kb_[NKB][8], vb[NKB][8];  // B of S = Q K^T and of dP = dO V^T: rows j0 + x of K, V
#pragma unroll
  for (int kb = 0; kb < NKB; ++kb) {
    ld8<S16>(K, head + (size_t)key * HS + 16 * kb + 8 * lk, kb_[kb]);
    ld8<S16>(V, head + (size_t)key * HS + 16 * kb + 8 * lk, vb[kb]);
  }
  Split3 ks[X3 ? NKB : 1], vs[X3 ? NKB : 1];
  if constexpr (X3)
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      ks[kb] = split3(kb_[kb]);
      vs[kb] = split3(vb[kb]);
    }
  v16f dvt[NN], dkt[NN];  // dV^T, dK^T: lane = key, rows = head dims
#pragma unroll
  for (int n = 0; n < NN; ++n) {
    dvt[n] = v16f{0};
    dkt[n] = v16f{0};
  }
  const int first = CAUSAL ? kt : 0;
  // f32: query tile it of Q and dO goes through LDS (rows padded to HS + 4
  // floats): one 16-byte global load per 4 floats, and both orientations
  // (rows for S and dP, columns for dV^T = dO^T P and dK^T = Q^T dS) read
  // back from LDS.  Under bf16 the products are too short to hide the
  // staging's round trip: there the operands come straight from L2 (the LDS
  // form measured 3 % faster at T = 256 but 3-20 % slower at T = 1024-4096).
  constexpr bool STAGE = !BF;
  static_assert(W == 1 || STAGE, "several key tiles per workgroup share the f32 staging");
  constexpr int LD = HS + 4, Q4 = HS / 4, PER = 32 * Q4 / (64 * W);
  __shared__ __attribute__((aligned(16))) float Qs[STAGE ? 32 * LD : 1], Os[STAGE ? 32 * LD : 1];
  // W > 1: the workgroup's query tiles start at its first wave's, and tile
  // it + 1's loads (a 1 / W share per thread) are issued before tile it's
  // products
  const int wg_first = W == 1 ? first : (CAUSAL ? W * (kt / W) : 0);
  v4f qf[W > 1 ? PER : 1], of[W > 1 ? PER : 1];
  if constexpr (W > 1)
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int f = threadIdx.x + 64 * W * u;
      qf[u] = ld4<S16>(Q, head + (size_t)(32 * wg_first + f / Q4) * HS + 4 * (f % Q4));
      of[u] = *reinterpret_cast<const v4f*>(head_row(dO, bh, H, T, ldo, HS, 32 * wg_first + f / Q4) + 4 * (f % Q4));
    }
  for (int it = wg_first; it < NT; ++it) {
    const int i0 = 32 * it;
    v16f s = v16f{0}, dp = v16f{0};
    if constexpr (STAGE && W > 1) {
      __syncthreads();  // every wave's reads of the last tile are done
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        const int f = threadIdx.x + 64 * W * u;
        *reinterpret_cast<v4f*>(Qs + (f / Q4) * LD + 4 * (f % Q4)) = qf[u];
        *reinterpret_cast<v4f*>(Os + (f / Q4) * LD + 4 * (f % Q4)) = of[u];
      }
      __syncthreads();  // this tile is visible to every wave
      if (it + 1 < NT)  // in flight during this tile's products
#pragma unroll
        for (int u = 0; u < PER; ++u) {
          const int f = threadIdx.x + 64 * W * u;
          qf[u] = ld4<S16>(Q, head + (size_t)(i0 + 32 + f / Q4) * HS + 4 * (f % Q4));
          of[u] = *reinterpret_cast<const v4f*>(head_row(dO, bh, H, T, ldo, HS, i0 + 32 + f / Q4) + 4 * (f % Q4));
        }
      if (it < first) continue;  // before this wave's diagonal: the barriers only
    }
    if constexpr (STAGE) {
      if constexpr (W == 1) {
        v4f qn[PER], on[PER];
#pragma unroll
        for (int u = 0; u < PER; ++u) {
          const int f = lane + 64 * u;
          qn[u] = ld4<S16>(Q, head + (size_t)(i0 + f / Q4) * HS + 4 * (f % Q4));
          on[u] = *reinterpret_cast<const v4f*>(head_row(dO, bh, H, T, ldo, HS, i0 + f / Q4) + 4 * (f % Q4));
        }
        wave_lds_sync();  // the last tile's reads of Qs and Os are done
#pragma unroll
        for (int u = 0; u < PER; ++u) {
          const int f = lane + 64 * u;
          *reinterpret_cast<v4f*>(Qs + (f / Q4) * LD + 4 * (f % Q4)) = qn[u];
          *reinterpret_cast<v4f*>(Os + (f / Q4) * LD + 4 * (f % Q4)) = on[u];
        }
        wave_lds_sync();  // this tile's stores are visible to every lane
      }
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        float qa[8], oa[8];  // A: rows perm_row(x) of Q_i, dO_i
        load8(Qs + perm_row(x) * LD + 16 * kb + 8 * lk, qa);
        load8(Os + perm_row(x) * LD + 16 * kb + 8 * lk, oa);
        if constexpr (X3) {
          s = x3_one<false>(split3(qa), ks[kb], s);
          dp = x3_one<false>(split3(oa), vs[kb], dp);
        } else {
          s = slab<BF>(qa, kb_[kb], s);
          dp = slab<BF>(oa, vb[kb], dp);
        }
      }
    } else {
      const int qrow = i0 + perm_row(x);
      const float* dorow = head_row(dO, bh, H, T, ldo, HS, qrow);
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        float qa[8], oa[8];  // A: rows perm_row(x) of Q_i, dO_i
        ld8<S16>(Q, head + (size_t)qrow * HS + 16 * kb + 8 * lk, qa);
        load8(dorow + 16 * kb + 8 * lk, oa);
        s = slab<BF>(qa, kb_[kb], s);
        dp = slab<BF>(oa, vb[kb], dp);
      }
    }
    // lane = key j0 + x, register r = query i0 + perm_index(r, lk)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float Lq[8], Dq_[8];
      load8(lseh + i0 + 16 * h + 8 * lk, Lq);
      load8(dsh + i0 + 16 * h + 8 * lk, Dq_);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int r = 8 * h + e;
        const bool masked = CAUSAL && key > i0 + perm_index(r, lk);
        const float p = masked ? 0.0f : expf(s[r] * sc - Lq[e]);
        const float diff = dp[r] - Dq_[e];
        const float dx = p * diff;
        s[r] = p;
        dp[r] = dx * sc;
      }
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float pb[8], db[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pb[e] = s[8 * h + e];
        db[e] = dp[8 * h + e];
      }
      Split3 pbs, dbs;
      if constexpr (X3) {
        pbs = split3(pb);
        dbs = split3(db);
      }
#pragma unroll
      for (int n = 0; n < NN; ++n) {
        float oa[8], qa[8];  // A of dV^T = dO^T P and dK^T = Q^T dS: [i0 + 16 h + 8 lk + e][32 n + x]
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if constexpr (STAGE) {
            const int q = 16 * h + 8 * lk + e;
            oa[e] = Os[q * LD + 32 * n + x];
            qa[e] = Qs[q * LD + 32 * n + x];
          } else {
            const int q = i0 + 16 * h + 8 * lk + e;
            oa[e] = head_row(dO, bh, H, T, ldo, HS, q)[32 * n + x];
            qa[e] = ld1<S16>(Q, head + (size_t)q * HS + 32 * n + x);
          }
        }
        if constexpr (X3) {
          dvt[n] = x3_one<false>(split3(oa), pbs, dvt[n]);
          dkt[n] = x3_one<false>(split3(qa), dbs, dkt[n]);
        } else {
          dvt[n] = slab<BF>(oa, pb, dvt[n]);
          dkt[n] = slab<BF>(qa, db, dkt[n]);
        }
      }
    }
  }
  // dV[j0 + x][32 n + 8 g + 4 lk + c] = dvt[n][4 g + c] (+ Dv), dK likewise
  // (the addends, where given, are all loaded before the first add)
  v4f av[NN][4], ak[NN][4];
#pragma unroll
  for (int n = 0; n < NN; ++n)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const size_t off = head + (size_t)key * HS + 32 * n + 8 * g + 4 * lk;
      if (!S16 && Dv) av[n][g] = *reinterpret_cast<const v4f*>(Dv + off);
      if (!S16 && Dk) ak[n][g] = *reinterpret_cast<const v4f*>(Dk + off);
    }
#pragma unroll
  for (int n = 0; n < NN; ++n)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const size_t off = head + (size_t)key * HS + 32 * n + 8 * g + 4 * lk;
      v4f wv, wk;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        wv[c] = dvt[n][4 * g + c];
        wk[c] = dkt[n][4 * g + c];
      }
      if (!S16 && Dv) wv = av[n][g] + wv;
      if (!S16 && Dk) wk = ak[n][g] + wk;
      st4<S16>(dV, off, wv);
      st4<S16>(dK, off, wk);
    }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

template <int HS, bool CAUSAL, bool BF, bool S16, bool X3 = false>
void fwd_launch(const float* Q, const float* K, const float* V, const float* scale, float* O, int ldo, int H,
                float* lse, int T, int BH, hipStream_t s) {
  k_flash_fwd<HS, CAUSAL, BF, S16, X3><<<(unsigned)(T / 32 * BH), 64, 0, s>>>(Q, K, V, scale, O, ldo, H, lse, T, BH);
}

template <int HS, bool CAUSAL, bool BF, bool S16, bool X3 = false>
void bwd_launch(const FlashBwd& a, int ldo, int H, int T, int BH, hipStream_t s) {
  const unsigned grid = (unsigned)(T / 32 * BH);
  // Split products at T >= 1024: four query (key) tiles per workgroup (dQ pass 4-7 %
  // faster at T = 1024 ... 4096; at T = 256 a head has two groups, the short
  // one's waves mostly wait at its barriers, and it measured 5 % slower, two
  // tiles per workgroup 3 % slower).
  bool grouped = false;
  if constexpr (X3) grouped = T / 32 >= 32 && (T / 32) % 4 == 0;
  if constexpr (X3) {
    if (grouped)
      k_flash_bwd_dq<HS, CAUSAL, BF, S16, X3, 4><<<grid / 4, 256, 0, s>>>(a.Q, a.K, a.V, a.O, a.dO, ldo, H, a.lse,
                                                                          a.scale, a.dQ, a.Dq, a.dsum, T, BH);
  }
  if (!grouped)
    k_flash_bwd_dq<HS, CAUSAL, BF, S16, X3><<<grid, 64, 0, s>>>(a.Q, a.K, a.V, a.O, a.dO, ldo, H, a.lse, a.scale,
                                                                 a.dQ, a.Dq, a.dsum, T, BH);
  if constexpr (X3) {
    if (grouped)
      k_flash_bwd_dkv<HS, CAUSAL, BF, S16, X3, 4><<<grid / 4, 256, 0, s>>>(a.Q, a.K, a.V, a.dO, ldo, H, a.lse, a.dsum,
                                                                           a.scale, a.dK, a.Dk, a.dV, a.Dv, T, BH);
  }
  if (!grouped)
    k_flash_bwd_dkv<HS, CAUSAL, BF, S16, X3><<<grid, 64, 0, s>>>(a.Q, a.K, a.V, a.dO, ldo, H, a.lse, a.dsum, a.scale,
                                                                  a.dK, a.Dk, a.dV, a.Dv, T, BH);
}

// precision: 0 f32 (FP32 MFMA), 1 bf16 MFMA on f32 storage, 2 bf16 MFMA on
// bf16 q, k, v (and their gradients), 3 f32 as split bf16 products
template <int HS, bool CAUSAL>
void fwd_prec(int prec, const float* Q, const float* K, const float* V, const float* scale, float* O, int ldo, int H,
              float* lse, int T, int BH, hipStream_t s) {
  if (prec == 3) fwd_launch<HS, CAUSAL, false, false, true>(Q, K, V, scale, O, ldo, H, lse, T, BH, s);
  else if (prec == 2) fwd_launch<HS, CAUSAL, true, true>(Q, K, V, scale, O, ldo, H, lse, T, BH, s);
  else if (prec == 1) fwd_launch<HS, CAUSAL, true, false>(Q, K, V, scale, O, ldo, H, lse, T, BH, s);
  else fwd_launch<HS, CAUSAL, false, false>(Q, K, V, scale, O, ldo, H, lse, T, BH, s);
}

template <bool CAUSAL>
void fwd_hs(size_t hs, int prec, const float* Q, const float* K, const float* V, const float* scale, float* O, int ldo,
            int H, float* lse, int T, int BH, hipStream_t s) {
  if (hs == 64) fwd_prec<64, CAUSAL>(prec, Q, K, V, scale, O, ldo, H, lse, T, BH, s);
  else fwd_prec<32, CAUSAL>(prec, Q, K, V, scale, O, ldo, H, lse, T, BH, s);
}

template <int HS, bool CAUSAL>
void bwd_prec(int prec, const FlashBwd& a, int ldo, int H, int T, int BH, hipStream_t s) {
  if (prec == 3) bwd_launch<HS, CAUSAL, false, false, true>(a, ldo, H, T, BH, s);
  else if (prec == 2) bwd_launch<HS, CAUSAL, true, true>(a, ldo, H, T, BH, s);
  else if (prec == 1) bwd_launch<HS, CAUSAL, true, false>(a, ldo, H, T, BH, s);
  else bwd_launch<HS, CAUSAL, false, false>(a, ldo, H, T, BH, s);
}

template <bool CAUSAL>
void bwd_hs(size_t hs, int prec, const FlashBwd& a, int ldo, int H, int T, int BH, hipStream_t s) {
  if (hs == 64) bwd_prec<64, CAUSAL>(prec, a, ldo, H, T, BH, s);
  else bwd_prec<32, CAUSAL>(prec, a, ldo, H, T, BH, s);
}

}  // namespace

bool flash_supported(size_t bh, size_t t, size_t hs) {
  return bh > 0 && t >= 32 && t % 32 == 0 && (hs == 32 || hs == 64) && (t / 32) * bh <= 0x7fffffffu &&
         bh * t * hs < (1ull << 40);
}

bool flash_fwd(const float* Q, const float* K, const float* V, const float* scale, float* O, size_t ldo, size_t heads,
               float* lse, size_t bh, size_t t, size_t hs, bool causal, bool bf16, hipStream_t s, bool qkv_bf16) {
  if (!flash_supported(bh, t, hs) || heads == 0 || bh % heads || ldo < hs * heads || ldo % 4) return false;
  if (!aligned16(Q) || !aligned16(K) || !aligned16(V) || !aligned16(O) || !lse || !scale) return false;
  const int T = (int)t, BH = (int)bh, l = (int)ldo, H = (int)heads;
  const int prec = qkv_bf16 ? 2 : bf16 ? 1 : gemm_f32_split() ? 3 : 0;
  if (causal) fwd_hs<true>(hs, prec, Q, K, V, scale, O, l, H, lse, T, BH, s);
  else fwd_hs<false>(hs, prec, Q, K, V, scale, O, l, H, lse, T, BH, s);
  MALUS_HIP(hipGetLastError());
  return true;
}

bool flash_bwd(const FlashBwd& a, size_t ldo, size_t heads, size_t bh, size_t t, size_t hs, bool causal, bool bf16,
               hipStream_t s, bool qkv_bf16) {
  if (!flash_supported(bh, t, hs) || heads == 0 || bh % heads || ldo < hs * heads || ldo % 4) return false;
  for (const void* p : {(const void*)a.Q, (const void*)a.K, (const void*)a.V, (const void*)a.O, (const void*)a.dO,
                        (const void*)a.dQ, (const void*)a.dK, (const void*)a.dV, (const void*)a.lse,
                        (const void*)a.dsum})
    if (!p || !aligned16(p)) return false;
  if ((a.Dk && !aligned16(a.Dk)) || (a.Dv && !aligned16(a.Dv)) || !a.scale) return false;
  if (qkv_bf16 && (a.Dq || a.Dk || a.Dv)) return false;  // bf16 gradients take no addends
  const int T = (int)t, BH = (int)bh, l = (int)ldo, H = (int)heads;
  const int prec = qkv_bf16 ? 2 : bf16 ? 1 : gemm_f32_split() ? 3 : 0;
  if (causal) bwd_hs<true>(hs, prec, a, l, H, T, BH, s);
  else bwd_hs<false>(hs, prec, a, l, H, T, BH, s);
  MALUS_HIP(hipGetLastError());
  return true;
}

}  // namespace k
}  // namespace malus
