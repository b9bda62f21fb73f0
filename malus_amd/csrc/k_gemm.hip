// Batched FP32 GEMM on gfx950 matrix cores (v_mfma_f32_32x32x2_f32).
//
//   C[b] = op(A[b]) @ op(B[b]),  op(A) = A or A^T (A stored [K, M]),
//                                op(B) = B or B^T (B stored [N, K]).
//
// The transposed forms serve the matmul VJPs (dA = dC @ B^T, dB = A^T @ dC)
// without materializing the transposes the reference builds with permute
// kernels (matmul_bwd.ml:15-29); the values are identical because a
// transpose is an exact copy.
//
// Tiling: 256 threads = 4 waves in a 2x2 grid; each wave owns TM x TN
// MFMA 32x32 accumulators, so the block tile is (64 TM) x (64 TN) with
// BK = 16.  Operand tiles are staged in LDS in their global orientation
// (see Tile), double-buffered with one barrier per K step; all MFMA operand
// fragments of a K step are read from LDS before its MFMAs issue, so LDS
// latency stays off the matrix pipe.  The host picks TM x TN and a K split
// per shape from a cost model of the busiest CU (256 CUs, the variant's
// occupancy from the runtime, padding waste of partial tiles).  Long-K
// shapes with few output tiles (the weight-gradient GEMMs, K = tokens)
// split K across workgroups and reduce the partials in split order; the
// split depends only on the shape, so results are deterministic.  Tile ids
// are remapped so consecutive tiles of one output row land on the same XCD
// (shared L2).
//
// MFMA lane layout (verified on gfx950): A[i][k] from lane i + 32k,
// B[k][j] from lane j + 32k, D register r of lane l holds
// D[8*(r/4) + 4*(l/32) + r%4][l%32].
#include <cstdlib>
#include <cstring>

#include "k_gemm_dma.h"

namespace malus {
namespace k {
namespace {

// One operand's tile: BX rows of its free dimension x (m for A, n for B) by
// BK of k, staged in LDS in the operand's global orientation, so staging
// never transposes:
//   KC (k-contiguous: A as [M][K], B^T as [N][K]) -> LDS [x][BK + 4];
//   XC (x-contiguous: A^T as [K][M], B as [K][N]) -> LDS [k][BX + 4].
// MFMA step s (0..7) of a K step gives lane (i, h) = (lane % 32, lane / 32)
// the element k = 8h + s, for A and B alike (any bijection of k works as
// long as both operands use the same one).  A KC lane then reads its 8 k
// values with two 128-bit LDS reads (row stride 20 floats: 8 lanes of a
// 128-bit phase hit disjoint banks); an XC lane reads one float per step,
// 32 consecutive floats per half-wave.
template <int BX, bool KC, bool VEC>
struct Tile {
  static constexpr int LD = KC ? BK + 4 : BX + 4;
  static constexpr int SIZE = KC ? BX * LD : BK * LD;
  static constexpr int NV = BX * BK / 4 / 256;  // float4 per thread
  static constexpr int NS = BX * BK / 256;      // floats per thread
  float r[NS];

  // Rows x0.. and k0.. of the operand P (row stride ld); x >= X or k >= klim
  // read as zero.
  __device__ __forceinline__ void load(const float* __restrict__ P, int X, long ld, int klim, int x0, int k0) {
    const int t = threadIdx.x;
    if (VEC) {
#pragma unroll
      for (int q = 0; q < NV; ++q) {
        const int idx = t + 256 * q;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (KC) {
          const int x = x0 + idx / (BK / 4), k = k0 + 4 * (idx % (BK / 4));
          if (x < X && k < klim) v = *reinterpret_cast<const float4*>(P + (size_t)x * ld + k);
        } else {
          const int k = k0 + idx / (BX / 4), x = x0 + 4 * (idx % (BX / 4));
          if (k < klim && x < X) v = *reinterpret_cast<const float4*>(P + (size_t)k * ld + x);
        }
        r[4 * q] = v.x; r[4 * q + 1] = v.y; r[4 * q + 2] = v.z; r[4 * q + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int q = 0; q < NS; ++q) {
        const int e = t + 256 * q;
        float v = 0.f;
        if (KC) {
          const int x = x0 + e / BK, k = k0 + e % BK;
          if (x < X && k < klim) v = P[(size_t)x * ld + k];
        } else {
          const int k = k0 + e / BX, x = x0 + e % BX;
          if (k < klim && x < X) v = P[(size_t)k * ld + x];
        }
        r[q] = v;
      }
    }
  }

  __device__ __forceinline__ void store(float* __restrict__ S) const {
    const int t = threadIdx.x;
    if (VEC) {
#pragma unroll
      for (int q = 0; q < NV; ++q) {
        const int idx = t + 256 * q;
        const int off = KC ? (idx / (BK / 4)) * LD + 4 * (idx % (BK / 4)) : (idx / (BX / 4)) * LD + 4 * (idx % (BX / 4));
        *reinterpret_cast<float4*>(S + off) = make_float4(r[4 * q], r[4 * q + 1], r[4 * q + 2], r[4 * q + 3]);
      }
    } else {
#pragma unroll
      for (int q = 0; q < NS; ++q) {
        const int e = t + 256 * q;
        S[KC ? (e / BK) * LD + e % BK : (e / BX) * LD + e % BX] = r[q];
      }
    }
  }

  // The 8 MFMA-step values of this lane for tile rows xw .. xw + 31.
  __device__ __forceinline__ static void frag(const float* __restrict__ S, int xw, float f[8]) {
    const int lane = threadIdx.x & 63, i = lane & 31, h = lane >> 5;
    if (KC) {
      const float4* p = reinterpret_cast<const float4*>(S + (xw + i) * LD + 8 * h);
      const float4 a = p[0], b = p[1];
      f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
      f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    } else {
#pragma unroll
      for (int s = 0; s < 8; ++s) f[s] = S[(8 * h + s) * LD + xw + i];
    }
  }
};

// grid: x = output tiles (XCD-remapped), y = K splits, z = batch.
// Split s writes its partial tile to C + s * split_stride.
template <int TM, int TN, bool TA, bool TB, bool VA, bool VB, bool BF = false>
__global__ __launch_bounds__(256, 2) void k_sgemm(const float* __restrict__ A, const float* __restrict__ B,
                                                  float* __restrict__ C, int M, int N, int K, long sA, long sB, long sC,
                                                  int k_chunk, int tiles_n, long split_stride,
                                                  const float* __restrict__ D) {
  constexpr int BM = 64 * TM, BN = 64 * TN;
  using TileA = Tile<BM, !TA, VA>;  // A [M][K] is k-contiguous
  using TileB = Tile<BN, TB, VB>;   // B^T [N][K] is k-contiguous
  __shared__ __attribute__((aligned(16))) float As[2][TileA::SIZE];
  __shared__ __attribute__((aligned(16))) float Bs[2][TileB::SIZE];

  const int nt = gridDim.x;
  int tile = blockIdx.x;
  if ((nt & 7) == 0) tile = (tile & 7) * (nt >> 3) + (tile >> 3);  // XCD-contiguous tile ranges
  const int tm = tile / tiles_n, tn = tile % tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;
  const int b = blockIdx.z;
  A += (size_t)b * sA;
  B += (size_t)b * sB;
  C += (size_t)b * sC + (size_t)blockIdx.y * split_stride;
  if (D) D += (size_t)b * sC;
  const int kbeg = blockIdx.y * k_chunk;
  const int kend = min(K, kbeg + k_chunk);
  const long lda = TA ? M : K, ldb = TB ? K : N;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = (wave >> 1) * 32 * TM, wn = (wave & 1) * 32 * TN;
  const int li = lane & 31, lk = lane >> 5;

  v16f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = v16f{0};

  TileA la;
  TileB lb;
  const int nk = (kend - kbeg + BK - 1) / BK;
  if (nk > 0) {
    la.load(A, M, lda, kend, m0, kbeg);
    lb.load(B, N, ldb, kend, n0, kbeg);
    la.store(As[0]);
    lb.store(Bs[0]);
  }
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      la.load(A, M, lda, kend, m0, kbeg + (kt + 1) * BK);
      lb.load(B, N, ldb, kend, n0, kbeg + (kt + 1) * BK);
    }
    float fa[TM][8], fb[TN][8];
#pragma unroll
    for (int i = 0; i < TM; ++i) TileA::frag(As[cur], wm + 32 * i, fa[i]);
#pragma unroll
    for (int j = 0; j < TN; ++j) TileB::frag(Bs[cur], wn + 32 * j, fb[j]);
    __builtin_amdgcn_sched_barrier(0);  // keep every fragment read ahead of the MFMA chain
    mfma_kstep<TM, TN, BF>(fa, fb, acc);
    if (more) {
      la.store(As[cur ^ 1]);
      lb.store(Bs[cur ^ 1]);
    }
    __syncthreads();
  }

  // epilogue: D register r of lane l -> row 8*(r/4) + 4*(l/32) + r%4, col l%32
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = n0 + wn + 32 * j + li;
      if (n < N) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * lk + (r & 3);
          if (m < M) C[(size_t)m * N + n] = D ? D[(size_t)m * N + n] + acc[i][j][r] : acc[i][j][r];
        }
      }
    }
}


// C[i] = sum over splits s (in order) of partial[s * mn + i], then + D[i]
// when an addend is given (the same rounding as adding to the stored sum).
__global__ __launch_bounds__(256) void k_split_reduce(const float* __restrict__ partial, float* __restrict__ C, size_t mn,
                                                      int nsplit, const float* __restrict__ D) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < mn; i += stride) {
    float acc = partial[i];
    for (int s = 1; s < nsplit; ++s) acc += partial[(size_t)s * mn + i];
    C[i] = D ? D[i] + acc : acc;
  }
}

// float4 form of k_split_reduce (same per-element order): eight partial
// loads are in flight before their adds, and 64-thread workgroups spread the
// few thousand float4 columns of a weight gradient over every CU.
typedef float v4f_t __attribute__((ext_vector_type(4)));
// blockIdx.y = group g of a grouped launch: its partials follow group
// g - 1's (nsplit * mn4 each) and it writes out.c[g].
struct SplitOut { v4f_t* c[3]; };
__global__ __launch_bounds__(64) void k_split_reduce4(const v4f_t* __restrict__ partial, SplitOut out, size_t mn4,
                                                      int nsplit, const v4f_t* __restrict__ D) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  partial += (size_t)blockIdx.y * nsplit * mn4;
  v4f_t* __restrict__ C = out.c[blockIdx.y];
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < mn4; i += stride) {
    v4f_t acc = partial[i];
    int s = 1;
    for (; s + 7 < nsplit; s += 8) {
      v4f_t t[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) t[u] = partial[(size_t)(s + u) * mn4 + i];
#pragma unroll
      for (int u = 0; u < 8; ++u) acc += t[u];
    }
    if (s < nsplit) {  // the last (at most 7) partials, also loaded before their adds
      v4f_t t[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (s + u < nsplit) t[u] = partial[(size_t)(s + u) * mn4 + i];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (s + u < nsplit) acc += t[u];
    }
    C[i] = D ? D[i] + acc : acc;
  }
}

// ---- kernel table -----------------------------------------------------------
struct TileCfg { int tm, tn; };
constexpr TileCfg kTiles[] = {{2, 3}, {2, 2}, {2, 1}, {1, 2}, {1, 1}};
constexpr int kNumTiles = sizeof(kTiles) / sizeof(kTiles[0]);

// Variant code: bit 14 = split f32 products, bits 13..9 = GemmLayouts::io
// (bf16-stored operands and split copies, the instances of k_gemm_io*.hip),
// bit 8 = bf16 MFMA (autocast), bit 7 =
// grouped accumulation, bit 6 = GELU epilogues, bit 5 = mapped operands,
// bit 4 = LDS-DMA path, bits 3..0 = transA, transB, vecA, vecB.
constexpr int kVarBf16 = 256;
constexpr int kVarIoShift = 9;
constexpr int kVarX3 = 1 << 14;  // f32 product as split bf16 pieces (LDS-DMA kernels)
constexpr int kVarCount = 1 << 15;
inline int variant(bool ta, bool tb, bool va, bool vb, bool dma) {
  return (dma << 4) | (ta << 3) | (tb << 2) | (va << 1) | (int)vb;
}

template <int TM, int TN, bool TA, bool TB, bool BF>
const void* kernel_of_reg(int v) {
  const bool va = v & 2, vb = v & 1;
  if (va && vb) return reinterpret_cast<const void*>(&k_sgemm<TM, TN, TA, TB, true, true, BF>);
  if (va) return reinterpret_cast<const void*>(&k_sgemm<TM, TN, TA, TB, true, false, BF>);
  if (vb) return reinterpret_cast<const void*>(&k_sgemm<TM, TN, TA, TB, false, true, BF>);
  return reinterpret_cast<const void*>(&k_sgemm<TM, TN, TA, TB, false, false, BF>);
}

// P: 0 f32 MFMA, 1 bf16 MFMA (autocast), 2 the f32 product as split bf16
// pieces (LDS-DMA kernels; the register-staged ones stay on the f32 MFMA)
template <int TM, int TN, bool TA, bool TB, int P>
const void* kernel_of(int v) {
  constexpr bool BF = P != 0, X3 = P == 2;
  if (v & 128) {  // grouped accumulation: mapped NT (the head projections' dA)
    if constexpr (!TA && TB) return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, false, true, true, 3, BF, 0, X3>);
    return nullptr;
  }
  if (v & 64) {  // GELU epilogues: dense NN (forward) and NT (the VJP's dA)
    if constexpr (!TA && !TB)
      return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, false, false, false, 1, BF, 0, X3>);
    if constexpr (!TA && TB) return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, false, true, false, 2, BF, 0, X3>);
    return nullptr;
  }
  if (v & 32) return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, TA, TB, true, 0, BF, 0, X3>);
  if (v & 16) return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, TA, TB, false, 0, BF, 0, X3>);
  return kernel_of_reg<TM, TN, TA, TB, P == 1>(v);
}

template <int TM, int TN, int P>
const void* kernel_of_layout(int v) {
  const bool ta = v & 8, tb = v & 4;
  if (!ta && !tb) return kernel_of<TM, TN, false, false, P>(v);
  if (!ta && tb) return kernel_of<TM, TN, false, true, P>(v);
  if (ta && !tb) return kernel_of<TM, TN, true, false, P>(v);
  return kernel_of<TM, TN, true, true, P>(v);
}

template <int P>
const void* kernel_for_prec(int ti, int v) {
  switch (ti) {
    case 0: return kernel_of_layout<2, 3, P>(v);
    case 1: return kernel_of_layout<2, 2, P>(v);
    case 2: return kernel_of_layout<2, 1, P>(v);
    case 3: return kernel_of_layout<1, 2, P>(v);
    default: return kernel_of_layout<1, 1, P>(v);
  }
}

const void* kernel_for(int ti, int v) {
  if ((v >> kVarIoShift) & 31) return gemm_io_kernel(ti, v);
  if (v & kVarX3) return kernel_for_prec<2>(ti, v);
  return (v & kVarBf16) ? kernel_for_prec<1>(ti, v) : kernel_for_prec<0>(ti, v);
}

// Co-resident workgroups per CU of each kernel variant (VGPR and LDS
// limited), from the runtime's occupancy calculator; cached per variant.
int occupancy(int ti, int v) {
  static int cache[kNumTiles][kVarCount];
  int& o = cache[ti][v];
  if (o == 0) {
    int n = 0;
    MALUS_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel_for(ti, v), 256, 0));
    o = n > 0 ? n : 1;
  }
  return o;
}

// ---- planning -----------------------------------------------------------------
// Relative MFMA efficiency of one workgroup of each tile, measured on the
// C5 shapes.  Register-staged: bigger tiles read fewer LDS fragments per
// MFMA and amortize the K-step barrier further.  LDS-DMA: staging costs no
// VGPRs or issue slots, and the 128-wide tiles keep up with the 256-wide
// ones while running more workgroups per CU.
inline double tile_base(int ti, bool dma) {
  static const double reg[kNumTiles] = {1.0, 0.97, 0.9, 0.9, 0.8};
  static const double lds_dma[kNumTiles] = {0.80, 0.85, 1.0, 1.0, 0.99};
  return dma ? lds_dma[ti] : reg[ti];
}
// Matrix-pipe utilization of a CU running `conc` workgroups at once (one
// workgroup is one wave per SIMD, which cannot hide its own LDS latency).
inline double cu_util(int conc) { return conc <= 1 ? 0.75 : conc == 2 ? 0.92 : 1.0; }

struct Plan { int ti, nsplit, k_chunk; };

int g_forced_tile = -2;    // -2: read MALUS_GEMM_TILE once; -1: automatic
bool g_autocast = false;   // GEMM products in bf16 with f32 accumulation (autocast scope)
int g_split_target = 0;    // workgroups a split-K launch aims for; 0: model
bool g_allow_dma = true;   // LDS-DMA path where the shape allows it
int g_f32_x3 = -1;         // f32 GEMMs as split bf16 products; -1: read MALUS_F32_GEMM once

// Default on; MALUS_F32_GEMM=fp32 starts the process on the FP32 MFMA.
bool f32_x3() {
  if (g_f32_x3 < 0) {
    const char* e = getenv("MALUS_F32_GEMM");
    g_f32_x3 = e && !strcmp(e, "fp32") ? 0 : 1;
  }
  return g_f32_x3 == 1;
}

// Pick the tile and the K split with the smallest modelled time: the
// busiest CU's MFMA work (256 CUs at 75 % of 157.3 TFLOP/s, scaled by the
// tile's efficiency and the CU's concurrency), plus the split-K partials'
// HBM round trip.  Long-K shapes with few output tiles (the weight-gradient
// GEMMs, K = tokens) split K so the grid fills the chip's workgroup slots.
// tri: A lower-triangular (GemmLayouts::tri_a); a tile row then runs on
// average (n + 1) / (2 n) of K for n tile rows, which favours short tiles.
// bf: the launch runs on the bf16 MFMA (autocast, or bf16-stored operands);
// x3: the f32 product as split bf16 pieces (LDS-DMA kernels); groups: the
// products one grouped launch runs side by side.
Plan plan_gemm(int batch, int M, int N, int K, int v, bool tri = false, int only_tile = -1, bool bf = false,
               bool x3 = false, int groups = 1) {
  if (g_forced_tile == -2) {  // MALUS_GEMM_TILE=TMxTN pins a tile (tuning sweeps)
    g_forced_tile = -1;
    if (const char* e = getenv("MALUS_GEMM_TILE"))
      for (int i = 0; i < kNumTiles; ++i) {
        char buf[8];
        snprintf(buf, sizeof(buf), "%dx%d", kTiles[i].tm, kTiles[i].tn);
        if (!strcmp(buf, e)) g_forced_tile = i;
      }
  }
  constexpr double kCuRate = 157.3e12 / 256 * 0.75;  // FLOP/s per CU
  constexpr double kHbm = 4.0e12;                     // B/s for the partials
  Plan best{0, 1, K};
  double best_t = 1e300;
  // Weight-gradient GEMMs on the LDS-DMA path (A^T @ dC, K = tokens): the
  // C5 sweep of tile x split put 128x64 / 64x128 tiles with ~512 workgroups
  // 10-17 % ahead of every other choice in f32, so the plan is fixed to
  // those.  Under autocast a bf16 K step is an eighth of the f32 one's MFMA
  // time, and the 128x192 tile (more MFMA work per staged byte) with the
  // cost model's split measured 10-20 % faster on the same shapes.
  const bool wgrad = (v & 16) && (v & 8) && batch == 1 && K >= 4096 && g_forced_tile < 0 && g_split_target == 0;
  // The split f32 product (six bf16 MFMAs per staged f32 slab) favours
  // wider tiles (fewer staged bytes per product) where the grid still fills
  // the chip.  Per call in the C5 step (kernel trace, 128x64 against the
  // wider tile): the three grouped q/k/v weight gradients 124 -> 114 us on
  // 128x128 with the cost model's split.  The single 384x384 weight
  // gradient (41 against 53 us), the 1536-wide ones, the GELU VJP (160
  // against 226 us: the wider tiles lose its epilogue prefetch) and the
  // K = 1536, N = 384 products keep the f32 plan (128x128 with a split of 2
  // gained 3-7 us a call before the forward GEMMs read split weights, and
  // measured 0.3 % slower on the step after); the GELU forward takes
  // 128x192 (153 -> 135 us) from the caller.
  const bool wgrad_bf = wgrad && (g_autocast || bf || (x3 && groups > 1));
  if (wgrad_bf) only_tile = x3 && !g_autocast && !bf ? 1 : 0;  // kTiles[0] = 128x192, kTiles[1] = 128x128
  // the occupancy the cost model sees: the split kernels' own for the wide
  // tiles picked above (it sets their K split), else the f32 kernels'
  const int occ_v = x3 && only_tile >= 0 ? (v & ~64) | kVarX3 : v & ~64;
  for (int ti = 0; ti < kNumTiles; ++ti) {
    if (g_forced_tile >= 0 && ti != g_forced_tile) continue;
    if (only_tile >= 0 && g_forced_tile < 0 && ti != only_tile) continue;
    const int bm = 64 * kTiles[ti].tm, bn = 64 * kTiles[ti].tn;
    if (wgrad && !wgrad_bf &&
        !((kTiles[ti].tm == 2 && kTiles[ti].tn == 1) || (kTiles[ti].tm == 1 && kTiles[ti].tn == 2)))
      continue;
    const long tiles = (long)((M + bm - 1) / bm) * ((N + bn - 1) / bn) * batch;
    const int occ = occupancy(ti, occ_v);
    int cand[3] = {1, 1, 1};
    if (batch == 1 && K >= 1024) {
      const int max_split = K / 512;  // >= 32 K steps per workgroup amortize its prologue and partial tile
      for (int w = 1; w <= 2; ++w) {
        long want = g_split_target > 0 ? g_split_target * w : wgrad && !wgrad_bf ? 512 : (long)w * occ * 256;
        long sp = want / tiles;
        cand[w] = (int)(sp < 1 ? 1 : sp > max_split ? max_split : sp);
      }
      if (wgrad && !wgrad_bf) cand[0] = cand[1];  // only the ~512-workgroup split
    }
    for (int c = 0; c < 3; ++c) {
      int kc = (K + cand[c] - 1) / cand[c];
      kc = (kc + BK - 1) / BK * BK;
      const int ns = (K + kc - 1) / kc;
      const long blocks = tiles * ns;
      const long per_cu = (blocks + 255) / 256;
      const int conc = (int)(per_cu < occ ? per_cu : occ);
      const int nrow = (M + bm - 1) / bm;
      const double kwork = tri ? kc * (nrow + 1.0) / (2.0 * nrow) : kc;
      double t = per_cu * 2.0 * bm * bn * kwork / (kCuRate * tile_base(ti, v & 16) * cu_util(conc));
      if (ns > 1) t += (ns + 1.0) * M * N * 4.0 / kHbm + 3e-6;
      if (t < best_t * 0.999) { best_t = t; best = Plan{ti, ns, kc}; }
    }
  }
  return best;
}

}  // namespace

namespace {

void trace_plan(int batch, int M, int N, int K, bool transA, bool transB, bool dma, const Plan& p, int v,
                const char* tag) {
  static const bool trace = getenv("MALUS_GEMM_TRACE") != nullptr;
  if (trace)
    fprintf(stderr, "malus gemm b%d %dx%dx%d t%d%d -> %s%s tile %dx%d occ %d split %d k_chunk %d\n", batch, M, N, K,
            transA, transB, dma ? "dma" : "reg", tag, 64 * kTiles[p.ti].tm, 64 * kTiles[p.ti].tn, occupancy(p.ti, v),
            p.nsplit, p.k_chunk);
}

// Sum the split-K partials into C (+ D) in split order, then return the
// partial buffer to the pool.
void split_reduce(float* partial, float* C, size_t mn, int nsplit, const float* D, hipStream_t s, size_t bucket,
                  bool release = true) {
  const bool vec = mn % 4 == 0 && (reinterpret_cast<uintptr_t>(C) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(partial) & 15) == 0 && (reinterpret_cast<uintptr_t>(D) & 15) == 0;
  if (vec) {
    size_t blocks = (mn / 4 + 63) / 64;
    if (blocks > 16384) blocks = 16384;
    const SplitOut out{{reinterpret_cast<v4f_t*>(C), nullptr, nullptr}};
    k_split_reduce4<<<(unsigned)blocks, 64, 0, s>>>(reinterpret_cast<const v4f_t*>(partial), out, mn / 4, nsplit,
                                                   reinterpret_cast<const v4f_t*>(D));
  } else {
    size_t blocks = (mn + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    k_split_reduce<<<(unsigned)blocks, 256, 0, s>>>(partial, C, mn, nsplit, D);
  }
  MALUS_HIP(hipGetLastError());
  if (release) pool_free(partial, bucket);
}

// One LDS-DMA launch (plus the split-K reduction); a split writes dense
// partials, so callers with a non-dense C pass split_ok = false.
// Returns the multiply-add work the launch runs (2 * rows * cols * k, with
// the k ranges a triangular A leaves).
double launch_dma(const float* A, const float* B, float* C, int batch, int M, int N, int K, bool transA, bool transB,
                  GemmLayouts L, hipStream_t s, const float* D, bool split_ok, bool mapped, float* E = nullptr,
                  int epi = 0) {
  // mapped operands run the MAP instance on the dense shape's plan, so a
  // mapped GEMM splits K exactly like its dense twin; bf16-stored operands
  // take the plan of the autocast GEMM on f32 copies of them, so the sums
  // run in the same order
  const int v = variant(transA, transB, false, false, true);
  // a split copy of B (kIoB3) feeds the split product; any other io mask
  // is bf16 storage, which runs on the bf16 MFMA
  const bool bf = g_autocast || (L.io & ~kIoB3), x3 = !bf && f32_x3();
  if ((L.io & kIoB3) && !x3) fail("malus: gemm: a split copy of B needs split f32 products (io mask %d)", L.io);
  const int vb = (epi ? v | 64 : mapped ? v | 32 : v) | (bf ? kVarBf16 : 0) | (L.io << kVarIoShift) | (x3 ? kVarX3 : 0);
  const void* fn = kernel_for(0, vb);
  if (!fn) fail("malus: gemm: no kernel for epilogue %d with transA=%d transB=%d and bf16 storage mask %d", epi, transA,
                transB, L.io);
  if ((L.io & kIoC16) && D) fail("malus: gemm: a bf16 output takes no addend");
  // Under autocast the GELU GEMM (h = x W1, K = 384, a 3072-workgroup grid
  // at 128x64) measured 20 % faster on 128x192 tiles.
  // The GELU forward GEMM takes 128x192 tiles under autocast, and with split
  // products where that still gives 512 workgroups (C5's 16384 x 1536).
  const bool gelu_wide = epi == 1 && (bf || (x3 && (long)((M + 127) / 128) * ((N + 191) / 192) * batch >= 512));
  Plan p = plan_gemm(batch, M, N, K, v | (x3 && epi ? 64 : 0), mapped && L.tri_a, gelu_wide ? 0 : -1, bf, x3);
  const char* tag = mapped ? " mapped" : "";
  if ((!split_ok || epi || (L.io & kIoC16)) && p.nsplit > 1) {
    p.nsplit = 1;
    p.k_chunk = K;
  }
  trace_plan(batch, M, N, K, transA, transB, true, p, v, tag);
  const int bm = 64 * kTiles[p.ti].tm, bn = 64 * kTiles[p.ti].tn;
  const int tiles_n = (N + bn - 1) / bn, tiles = ((M + bm - 1) / bm) * tiles_n;
  int nsplit = p.nsplit, k_chunk = p.k_chunk;
  const size_t mn = (size_t)M * N;
  size_t bucket = 0;
  float* dst = C;
  if (nsplit > 1) {
    dst = static_cast<float*>(pool_alloc(mn * nsplit * sizeof(float), &bucket));
    L.c = dense_layout(N, 0);
  }
  long split_stride = nsplit > 1 ? (long)mn : 0;
  const float* Dk = nsplit > 1 ? nullptr : D;  // split-K applies the addend in the reduction
  void* args[] = {&A, &B, &dst, &M, &N, &K, &L, &k_chunk, const_cast<int*>(&tiles_n), &split_stride, &Dk, &E};
  fn = kernel_for(p.ti, vb);
  MALUS_HIP(hipLaunchKernel(fn, dim3((unsigned)tiles, (unsigned)nsplit, (unsigned)batch), dim3(256), args, 0, s));
  if (nsplit > 1) split_reduce(dst, C, mn, nsplit, D, s, bucket);
  if (!(mapped && L.tri_a)) return 2.0 * batch * (double)M * N * K;
  double rk = 0;  // sum over tile rows of rows * k range
  for (int m0 = 0; m0 < M; m0 += bm) {
    const int rows = M - m0 < bm ? M - m0 : bm;
    const int klen = transA ? K - m0 : (m0 + bm < K ? m0 + bm : K);
    rk += (double)rows * klen;
  }
  return 2.0 * batch * (double)N * rk;
}

bool map_contig(const GemmMap& f, int run) { return f.s0 == 1 && (f.div == 0 || f.div % run == 0); }
bool map_k16(const GemmMap& f) { return f.div == 0 || f.div % 16 == 0; }
// largest offset the map reaches for x in [0, n)
long map_max(const GemmMap& f, long n) {
  if (n <= 0) return 0;
  if (!f.div) return (n - 1) * f.s0;
  const long q = (n - 1) / f.div, r = f.div - 1 < n - 1 ? f.div - 1 : n - 1;
  return q * f.s1 + r * f.s0;
}

}  // namespace

void gemm(const float* A, const float* B, float* C, int batch, int M, int N, int K, bool transA, bool transB, long sA,
          long sB, long sC, hipStream_t s, const float* D, int io) {
  if (batch <= 0 || M <= 0 || N <= 0) return;
  if (K <= 0) {  // empty inner dimension: all-zero result (metal.rs:837-839 falls to the CPU loop)
    fill(C, 0.0f, (size_t)batch * M * N, s);
    return;
  }
  if (batch > 65535) fail("malus: gemm batch %d exceeds 65535", batch);
  const long lda = transA ? M : K, ldb = transB ? K : N;
  const long ext_a = (long)(batch - 1) * sA + (long)M * K, ext_b = (long)(batch - 1) * sB + (long)K * N;
  // LDS-DMA path: whole 16-deep K slabs, 16-byte rows, 32-bit byte offsets
  // (a bf16 operand's x-contiguous rows: runs of 8 elements)
  const int xa = io & kIoA16 ? 8 : 4, xb = io & (kIoB16 | kIoB3) ? 8 : 4;
  const bool dma = K % 16 == 0 && (transA ? M % xa == 0 : true) && (transB ? true : N % xb == 0) &&
                   (size_t)ext_a * 4 < (1ull << 31) && (size_t)ext_b * ((io & kIoB3) ? 6 : 4) < (1ull << 31) &&
                   ((size_t)(batch - 1) * sC + (size_t)M * N) * 4 < (1ull << 31) && g_allow_dma;
  if (io & ~(kIoA16 | kIoB16 | kIoB3)) fail("malus: gemm: bf16 storage mask %d is not an operand mask", io);
  if (dma) {
    GemmLayouts L{dense_layout(lda, sA), dense_layout(ldb, sB), dense_layout(N, sC), (int)ext_a, (int)ext_b};
    L.io = io;
    launch_dma(A, B, C, batch, M, N, K, transA, transB, L, s, D, true, false);
    return;
  }
  if (io)
    fail("malus: gemm: bf16-stored operands need the LDS-DMA kernels (%dx%dx%d, transA=%d transB=%d: K %% 16, "
         "the contiguous dimension of a bf16 operand %% 8)", M, N, K, transA, transB);
  // float4 staging needs the contiguous dim of each operand to be a multiple of 4
  const bool va = transA ? (M % 4 == 0) : (K % 4 == 0);
  const bool vb = transB ? (K % 4 == 0) : (N % 4 == 0);
  const int v = variant(transA, transB, va, vb, false);
  const Plan p = plan_gemm(batch, M, N, K, v);
  trace_plan(batch, M, N, K, transA, transB, false, p, v, "");
  const int bm = 64 * kTiles[p.ti].tm, bn = 64 * kTiles[p.ti].tn;
  const int tiles_m = (M + bm - 1) / bm, tiles_n = (N + bn - 1) / bn;
  const int tiles = tiles_m * tiles_n;
  int nsplit = p.nsplit, k_chunk = p.k_chunk;
  const size_t mn = (size_t)M * N;
  size_t bucket = 0;
  float* dst = C;
  if (nsplit > 1) dst = static_cast<float*>(pool_alloc(mn * nsplit * sizeof(float), &bucket));
  long split_stride = nsplit > 1 ? (long)mn : 0;
  const float* Dk = nsplit > 1 ? nullptr : D;  // split-K applies the addend in the reduction
  void* args[] = {&A, &B, &dst, &M, &N, &K, &sA, &sB, &sC, &k_chunk, const_cast<int*>(&tiles_n), &split_stride, &Dk};
  MALUS_HIP(hipLaunchKernel(kernel_for(p.ti, v | (g_autocast ? kVarBf16 : 0)),
                            dim3((unsigned)tiles, (unsigned)nsplit, (unsigned)batch), dim3(256), args, 0, s));
  if (nsplit > 1) split_reduce(dst, C, mn, nsplit, D, s, bucket);
}

bool gemm_gelu(const float* A, const float* B, float* C, float* E, int M, int N, int K, bool transB, bool backward,
               hipStream_t s, const float* D, int io) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 16 || N % 4 || !g_allow_dma || (!backward && (D || transB)) ||
      (backward && !transB))
    return false;
  const long ext_a = (long)M * K, ext_b = (long)K * N;
  if ((size_t)ext_a * 4 >= (1ull << 31) || (size_t)ext_b * ((io & kIoB3) ? 6 : 4) >= (1ull << 31) ||
      (size_t)M * N * 4 >= (1ull << 31))
    return false;
  GemmLayouts L{dense_layout(K, 0), dense_layout(transB ? K : N, 0), dense_layout(N, 0), (int)ext_a, (int)ext_b};
  L.io = io;
  launch_dma(A, B, C, 1, M, N, K, false, transB, L, s, D, false, false, E, backward ? 2 : 1);
  return true;
}

namespace {
bool mapped_ok(int batch, int M, int N, int K, bool transA, bool transB, const GemmLayouts& L);
}

bool gemm_grouped(int M, int N, int K, bool transA, bool transB, const GemmLayouts& Lin, float* C, bool accumulate,
                  hipStream_t s, const float* D, double* flops) {
  if (Lin.ngroup < 1 || Lin.ngroup > 3 || Lin.tri_a || !mapped_ok(1, M, N, K, transA, transB, Lin)) return false;
  if (accumulate && !(!transA && transB)) return false;  // built for the projections' dA (NT) only
  GemmLayouts L = Lin;
  const int v = variant(transA, transB, false, false, true);
  const bool bf = g_autocast || (L.io & ~kIoB3), x3 = !bf && f32_x3();
  if ((L.io & kIoB3) && !x3) fail("malus: gemm_grouped: a split copy of B needs split f32 products");
  Plan p = plan_gemm(1, M, N, K, v, false, -1, bf, x3, L.ngroup);
  const bool c_dense = L.c.r.div == 0 && L.c.c.div == 0 && L.c.c.s0 == 1 && L.c.r.s0 == N;
  if (accumulate || !c_dense || (L.io & kIoC16)) {  // split partials are f32 and dense
    p.nsplit = 1;
    p.k_chunk = K;
  }
  if (!accumulate && !c_dense && g_forced_tile < 0) {
    // Separate groups without a split multiply the tile count by ngroup:
    // take the widest tile that still gives every CU three workgroups (the
    // q/k/v projections, 16384 x 384 x 384 x 3: 128 x 192 tiles run 9 %
    // faster than the single GEMM's 128 x 64).
    for (int ti = 0; ti < kNumTiles; ++ti) {
      const long tiles = (long)((M + 64 * kTiles[ti].tm - 1) / (64 * kTiles[ti].tm)) *
                         ((N + 64 * kTiles[ti].tn - 1) / (64 * kTiles[ti].tn)) * L.ngroup;
      if (N % (64 * kTiles[ti].tn) == 0 && tiles >= 3 * 256) {
        p.ti = ti;
        break;
      }
    }
  }
  static const bool trace = getenv("MALUS_GEMM_TRACE") != nullptr;
  if (trace)
    fprintf(stderr, "malus gemm b1 %dx%dx%d t%d%d -> dma grouped%d%s tile %dx%d occ %d split %d k_chunk %d\n", M, N, K,
            transA, transB, L.ngroup, accumulate ? " acc" : "", 64 * kTiles[p.ti].tm, 64 * kTiles[p.ti].tn,
            occupancy(p.ti, v), p.nsplit, p.k_chunk);
  const int bm = 64 * kTiles[p.ti].tm, bn = 64 * kTiles[p.ti].tn;
  const int tiles_n = (N + bn - 1) / bn, tiles = ((M + bm - 1) / bm) * tiles_n;
  int nsplit = p.nsplit, k_chunk = p.k_chunk;
  const size_t mn = (size_t)M * N;
  size_t bucket = 0;
  float* partial = nullptr;
  float* outs[3] = {L.gc[0], L.gc[1], L.gc[2]};
  if (nsplit > 1) {
    partial = static_cast<float*>(pool_alloc(mn * nsplit * L.ngroup * sizeof(float), &bucket));
    for (int g = 0; g < L.ngroup; ++g) L.gc[g] = partial + (size_t)g * nsplit * mn;
    L.c = dense_layout(N, 0);
  }
  long split_stride = nsplit > 1 ? (long)mn : 0;
  const float* Dk = accumulate ? D : nullptr;
  float* E = nullptr;
  float* Cp = accumulate ? C : L.gc[0];
  const float *A0 = L.ga[0], *B0 = L.gb[0];
  void* args[] = {&A0, &B0, &Cp, &M, &N, &K, &L, &k_chunk, const_cast<int*>(&tiles_n), &split_stride, &Dk, &E};
  const void* fn = kernel_for(p.ti, (accumulate ? v | 128 : v | 32) | (bf ? kVarBf16 : 0) | (L.io << kVarIoShift) |
                                        (x3 ? kVarX3 : 0));
  if (!fn) fail("malus: gemm_grouped: no kernel for transA=%d transB=%d and bf16 storage mask %d", transA, transB, L.io);
  MALUS_HIP(hipLaunchKernel(fn, dim3((unsigned)tiles, (unsigned)nsplit, accumulate ? 1u : (unsigned)L.ngroup), dim3(256),
                            args, 0, s));
  if (nsplit > 1) {
    bool vec = mn % 4 == 0;
    for (int g = 0; g < L.ngroup; ++g) vec = vec && (reinterpret_cast<uintptr_t>(outs[g]) & 15) == 0;
    if (vec) {  // one launch for every group's reduction
      SplitOut out{};
      for (int g = 0; g < L.ngroup; ++g) out.c[g] = reinterpret_cast<v4f_t*>(outs[g]);
      size_t blocks = (mn / 4 + 63) / 64;
      if (blocks > 16384) blocks = 16384;
      k_split_reduce4<<<dim3((unsigned)blocks, (unsigned)L.ngroup), 64, 0, s>>>(reinterpret_cast<const v4f_t*>(partial),
                                                                               out, mn / 4, nsplit, nullptr);
      MALUS_HIP(hipGetLastError());
    } else {
      for (int g = 0; g < L.ngroup; ++g) {
        size_t none = 0;
        split_reduce(L.gc[g], outs[g], mn, nsplit, nullptr, s, none, false);
      }
    }
    pool_free(partial, bucket);
  }
  if (flops) *flops = 2.0 * L.ngroup * (double)M * N * K;
  return true;
}

bool gemm_mapped(const float* A, const float* B, float* C, int batch, int M, int N, int K, bool transA, bool transB,
                 const GemmLayouts& L, hipStream_t s, const float* D, double* flops) {
  if (!mapped_ok(batch, M, N, K, transA, transB, L)) return false;
  if (L.tri_a && M != K) return false;
  const bool c_dense = L.c.r.div == 0 && L.c.c.div == 0 && L.c.c.s0 == 1 && L.c.r.s0 == N;
  const double f = launch_dma(A, B, C, batch, M, N, K, transA, transB, L, s, D, c_dense && batch == 1 && !L.tri_a, true);
  if (flops) *flops = f;
  return true;
}

namespace {
bool mapped_ok(int batch, int M, int N, int K, bool transA, bool transB, const GemmLayouts& L) {
  if (batch <= 0 || M <= 0 || N <= 0 || K <= 0 || batch > 65535 || K % 16 || !g_allow_dma) return false;
  // contiguous dimension of each stored operand: runs of 4 floats (16
  // bytes), of 8 elements for a bf16 operand
  const GemmMap& a_contig = L.a.c;  // A [M][K]: k;  A^T [K][M]: m
  const GemmMap& b_contig = L.b.c;  // B [K][N]: n;  B^T [N][K]: k
  const int ra = L.io & kIoA16 ? 8 : 4, rb = L.io & (kIoB16 | kIoB3) ? 8 : 4;
  if (!map_contig(a_contig, ra) || !map_contig(b_contig, rb)) return false;
  if (transA ? M % ra : 0) return false;
  if (transB ? 0 : N % rb) return false;
  const GemmMap& fak = transA ? L.a.r : L.a.c;
  const GemmMap& fbk = transB ? L.b.c : L.b.r;
  if (!map_k16(fak) || !map_k16(fbk)) return false;
  if (L.c.r.div % 32) return false;
  // every operand offset the kernels form stays below 2^31 bytes
  const long lim = (1l << 31) / 4;
  const long ea = map_max(L.a.b, batch) + map_max(L.a.r, transA ? K : M) + map_max(L.a.c, transA ? M : K) + 1;
  const long eb = map_max(L.b.b, batch) + map_max(L.b.r, transB ? N : K) + map_max(L.b.c, transB ? K : N) + 1;
  const long ec = map_max(L.c.b, batch) + map_max(L.c.r, (M + 127) / 128 * 128) + map_max(L.c.c, N) + 1;
  if (ea > L.ext_a || eb > L.ext_b || L.ext_a >= lim || L.ext_b >= lim || ec >= lim) return false;
  if ((L.io & kIoB3) && (long)L.ext_b * 6 >= (1l << 31)) return false;  // the three planes' byte offsets
  return true;
}
}  // namespace

}  // namespace k
}  // namespace malus

// Tuning knob: pin the GEMM block tile to (64 tm) x (64 tn); (0, 0) restores
// the automatic choice.  Unknown tiles are rejected.
extern "C" int malus_gemm_set_tile(int tm, int tn) {
  using namespace malus::k;
  if (tm == 0 && tn == 0) { g_forced_tile = -1; return 1; }
  for (int i = 0; i < kNumTiles; ++i)
    if (kTiles[i].tm == tm && kTiles[i].tn == tn) { g_forced_tile = i; return 1; }
  return 0;
}

// The autocast scope (docs/adr/0037-bf16-autocast.md:5-12: matmuls in bf16
// with f32 accumulation; parameters, gradients, optimizer state and
// reductions stay f32): while on, every GEMM launch rounds its operands to
// bf16 and runs the bf16 MFMA.  A `with autocast:` block turns it on at entry
// and restores the returned previous state at exit.
namespace malus {
namespace k {
bool autocast_on() { return g_autocast; }
}  // namespace k
}  // namespace malus

extern "C" int malus_autocast(int on) {
  const bool prev = malus::k::g_autocast;
  malus::k::g_autocast = on != 0;
  return prev ? 1 : 0;
}

// f32 GEMMs on the LDS-DMA kernels as split bf16 products (1) or on the
// f32 MFMA (0); returns the previous setting.
namespace malus {
namespace k {
bool gemm_f32_split() { return f32_x3(); }
}  // namespace k
}  // namespace malus

extern "C" int malus_gemm_set_f32_split(int on) {
  const int prev = malus::k::f32_x3() ? 1 : 0;
  malus::k::g_f32_x3 = on != 0 ? 1 : 0;
  return prev;
}

// Tuning knob: 0 keeps every GEMM on the register-staged path (for A/B
// comparisons); 1 (default) uses the LDS-DMA path where the shape allows.
extern "C" void malus_gemm_set_dma(int on) { malus::k::g_allow_dma = on != 0; }

// Tuning knob: the number of workgroups a split-K GEMM aims for (0 restores
// the cost model's choice).
extern "C" void malus_gemm_set_split(int target_blocks) {
  malus::k::g_split_target = target_blocks > 0 ? target_blocks : 0;
}
