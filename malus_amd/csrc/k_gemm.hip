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
// BK = 16.  Operand tiles are staged in LDS as [k][m] / [k][n] (every MFMA
// operand read is 32 consecutive floats per half-wave); global->LDS staging
// is double-buffered with one barrier per K step, and all MFMA operand
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

#include "common.h"

namespace malus {
namespace k {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int BK = 16, PAD = 4;

template <int BM, bool TA, bool VA>
struct ALoader {
  static constexpr int N4 = BM * BK / 4 / 256;  // float4 per thread
  static constexpr int NS = BM * BK / 256;      // scalars per thread
  static constexpr int LDS = BM + PAD;
  float r[NS];
  // Tile (m0.., k0..) of A.  K is the row stride of a row-major A ([M][K]);
  // k >= klim reads as zero.
  __device__ __forceinline__ void load(const float* __restrict__ A, int M, int K, int klim, int m0, int k0) {
    const int t = threadIdx.x;
    if (VA) {
#pragma unroll
      for (int q = 0; q < N4; ++q) {
        int idx = t + 256 * q;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (!TA) {
          int rr = idx >> 2, c4 = idx & 3;
          int m = m0 + rr, k = k0 + c4 * 4;
          if (m < M && k < klim) v = *reinterpret_cast<const float4*>(A + (size_t)m * K + k);
        } else {
          int kr = idx / (BM / 4), c4 = idx % (BM / 4);
          int k = k0 + kr, m = m0 + c4 * 4;
          if (k < klim && m < M) v = *reinterpret_cast<const float4*>(A + (size_t)k * M + m);
        }
        r[4 * q] = v.x; r[4 * q + 1] = v.y; r[4 * q + 2] = v.z; r[4 * q + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int q = 0; q < NS; ++q) {
        int e = t + 256 * q;
        float v = 0.f;
        if (!TA) {
          int rr = e >> 4, kk = e & 15;
          int m = m0 + rr, k = k0 + kk;
          if (m < M && k < klim) v = A[(size_t)m * K + k];
        } else {
          int kr = e / BM, mm = e % BM;
          int k = k0 + kr, m = m0 + mm;
          if (k < klim && m < M) v = A[(size_t)k * M + m];
        }
        r[q] = v;
      }
    }
  }
  __device__ __forceinline__ void store(float* __restrict__ As) const {
    const int t = threadIdx.x;
    if (VA) {
#pragma unroll
      for (int q = 0; q < N4; ++q) {
        int idx = t + 256 * q;
        if (!TA) {
          int rr = idx >> 2, c4 = idx & 3;
#pragma unroll
          for (int j = 0; j < 4; ++j) As[(c4 * 4 + j) * LDS + rr] = r[4 * q + j];
        } else {
          int kr = idx / (BM / 4), c4 = idx % (BM / 4);
          *reinterpret_cast<float4*>(As + kr * LDS + c4 * 4) = make_float4(r[4 * q], r[4 * q + 1], r[4 * q + 2], r[4 * q + 3]);
        }
      }
    } else {
#pragma unroll
      for (int q = 0; q < NS; ++q) {
        int e = t + 256 * q;
        if (!TA) As[(e & 15) * LDS + (e >> 4)] = r[q];
        else As[(e / BM) * LDS + (e % BM)] = r[q];
      }
    }
  }
};

// B is the same problem with (m, M, TA) replaced by (n, N, !TB): a
// transposed B ([N][K]) is stored like a row-major A.
template <int BN, bool TB, bool VB>
using BLoader = ALoader<BN, !TB, VB>;

// grid: x = output tiles (XCD-remapped), y = K splits, z = batch.
// Split s writes its partial tile to C + s * split_stride.
template <int TM, int TN, bool TA, bool TB, bool VA, bool VB>
__global__ __launch_bounds__(256, 2) void k_sgemm(const float* __restrict__ A, const float* __restrict__ B,
                                                  float* __restrict__ C, int M, int N, int K, long sA, long sB, long sC,
                                                  int k_chunk, int tiles_n, long split_stride) {
  constexpr int BM = 64 * TM, BN = 64 * TN;
  constexpr int LDA = BM + PAD, LDB = BN + PAD;
  __shared__ __attribute__((aligned(16))) float As[2][BK * LDA];
  __shared__ __attribute__((aligned(16))) float Bs[2][BK * LDB];

  const int nt = gridDim.x;
  int tile = blockIdx.x;
  if ((nt & 7) == 0) tile = (tile & 7) * (nt >> 3) + (tile >> 3);  // XCD-contiguous tile ranges
  const int tm = tile / tiles_n, tn = tile % tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;
  const int b = blockIdx.z;
  A += (size_t)b * sA;
  B += (size_t)b * sB;
  C += (size_t)b * sC + (size_t)blockIdx.y * split_stride;
  const int kbeg = blockIdx.y * k_chunk;
  const int kend = min(K, kbeg + k_chunk);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = (wave >> 1) * 32 * TM, wn = (wave & 1) * 32 * TN;
  const int li = lane & 31, lk = lane >> 5;

  v16f acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = v16f{0};

  ALoader<BM, TA, VA> la;
  BLoader<BN, TB, VB> lb;
  const int nk = (kend - kbeg + BK - 1) / BK;
  if (nk > 0) {
    la.load(A, M, K, kend, m0, kbeg);
    lb.load(B, N, K, kend, n0, kbeg);
    la.store(As[0]);
    lb.store(Bs[0]);
  }
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      la.load(A, M, K, kend, m0, kbeg + (kt + 1) * BK);
      lb.load(B, N, K, kend, n0, kbeg + (kt + 1) * BK);
    }
    const float* as = As[cur] + lk * LDA + wm + li;
    const float* bs = Bs[cur] + lk * LDB + wn + li;
    float fa[BK / 2][TM], fb[BK / 2][TN];
#pragma unroll
    for (int kk = 0; kk < BK / 2; ++kk) {
#pragma unroll
      for (int i = 0; i < TM; ++i) fa[kk][i] = as[2 * kk * LDA + 32 * i];
#pragma unroll
      for (int j = 0; j < TN; ++j) fb[kk][j] = bs[2 * kk * LDB + 32 * j];
    }
#pragma unroll
    for (int kk = 0; kk < BK / 2; ++kk)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[kk][i], fb[kk][j], acc[i][j], 0, 0, 0);
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
          if (m < M) C[(size_t)m * N + n] = acc[i][j][r];
        }
      }
    }
}

// C[i] = sum over splits s (in order) of partial[s * mn + i]
__global__ __launch_bounds__(256) void k_split_reduce(const float* __restrict__ partial, float* __restrict__ C, size_t mn,
                                                      int nsplit) {
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < mn; i += stride) {
    float acc = partial[i];
    for (int s = 1; s < nsplit; ++s) acc += partial[(size_t)s * mn + i];
    C[i] = acc;
  }
}

// ---- kernel table -----------------------------------------------------------
struct TileCfg { int tm, tn; };
constexpr TileCfg kTiles[] = {{2, 3}, {2, 2}, {2, 1}, {1, 2}, {1, 1}};
constexpr int kNumTiles = sizeof(kTiles) / sizeof(kTiles[0]);

template <int TM, int TN, bool TA, bool TB>
const void* kernel_of(bool va, bool vb) {
  if (va && vb) return reinterpret_cast<const void*>(&k_sgemm<TM, TN, TA, TB, true, true>);
  if (va) return reinterpret_cast<const void*>(&k_sgemm<TM, TN, TA, TB, true, false>);
  if (vb) return reinterpret_cast<const void*>(&k_sgemm<TM, TN, TA, TB, false, true>);
  return reinterpret_cast<const void*>(&k_sgemm<TM, TN, TA, TB, false, false>);
}

template <int TM, int TN>
const void* kernel_of_layout(bool ta, bool tb, bool va, bool vb) {
  if (!ta && !tb) return kernel_of<TM, TN, false, false>(va, vb);
  if (!ta && tb) return kernel_of<TM, TN, false, true>(va, vb);
  if (ta && !tb) return kernel_of<TM, TN, true, false>(va, vb);
  return kernel_of<TM, TN, true, true>(va, vb);
}

const void* kernel_for(int ti, bool ta, bool tb, bool va, bool vb) {
  switch (ti) {
    case 0: return kernel_of_layout<2, 3>(ta, tb, va, vb);
    case 1: return kernel_of_layout<2, 2>(ta, tb, va, vb);
    case 2: return kernel_of_layout<2, 1>(ta, tb, va, vb);
    case 3: return kernel_of_layout<1, 2>(ta, tb, va, vb);
    default: return kernel_of_layout<1, 1>(ta, tb, va, vb);
  }
}

// Co-resident workgroups per CU of each kernel variant (VGPR and LDS
// limited), from the runtime's occupancy calculator; cached per variant.
int occupancy(int ti, bool ta, bool tb, bool va, bool vb) {
  static int cache[kNumTiles][16];
  const int v = (ta << 3) | (tb << 2) | (va << 1) | (int)vb;
  int& o = cache[ti][v];
  if (o == 0) {
    int n = 0;
    MALUS_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel_for(ti, ta, tb, va, vb), 256, 0));
    o = n > 0 ? n : 1;
  }
  return o;
}

// ---- planning -----------------------------------------------------------------
// Relative MFMA efficiency of one workgroup of each tile (bigger tiles read
// fewer LDS fragments per MFMA and amortize the K-step barrier further).
inline double tile_base(int ti) {
  static const double e[kNumTiles] = {1.0, 0.97, 0.9, 0.9, 0.8};
  return e[ti];
}
// Matrix-pipe utilization of a CU running `conc` workgroups at once (one
// workgroup is one wave per SIMD, which cannot hide its own LDS latency).
inline double cu_util(int conc) { return conc <= 1 ? 0.75 : conc == 2 ? 0.92 : 1.0; }

struct Plan { int ti, nsplit, k_chunk; };

int g_forced_tile = -2;    // -2: read MALUS_GEMM_TILE once; -1: automatic
int g_split_target = 0;    // workgroups a split-K launch aims for; 0: model

// Pick the tile and the K split with the smallest modelled time: the
// busiest CU's MFMA work (256 CUs at 75 % of 157.3 TFLOP/s, scaled by the
// tile's efficiency and the CU's concurrency), plus the split-K partials'
// HBM round trip.  Long-K shapes with few output tiles (the weight-gradient
// GEMMs, K = tokens) split K so the grid fills the chip's workgroup slots.
Plan plan_gemm(int batch, int M, int N, int K, bool ta, bool tb, bool va, bool vb) {
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
  for (int ti = 0; ti < kNumTiles; ++ti) {
    if (g_forced_tile >= 0 && ti != g_forced_tile) continue;
    const int bm = 64 * kTiles[ti].tm, bn = 64 * kTiles[ti].tn;
    const long tiles = (long)((M + bm - 1) / bm) * ((N + bn - 1) / bn) * batch;
    const int occ = occupancy(ti, ta, tb, va, vb);
    int cand[3] = {1, 1, 1};
    if (batch == 1 && K >= 1024) {
      const int max_split = K / 512;  // >= 32 K steps per workgroup amortize its prologue and partial tile
      for (int w = 1; w <= 2; ++w) {
        long want = g_split_target > 0 ? g_split_target * w : (long)w * occ * 256;
        long sp = want / tiles;
        cand[w] = (int)(sp < 1 ? 1 : sp > max_split ? max_split : sp);
      }
    }
    for (int c = 0; c < 3; ++c) {
      int kc = (K + cand[c] - 1) / cand[c];
      kc = (kc + BK - 1) / BK * BK;
      const int ns = (K + kc - 1) / kc;
      const long blocks = tiles * ns;
      const long per_cu = (blocks + 255) / 256;
      const int conc = (int)(per_cu < occ ? per_cu : occ);
      double t = per_cu * 2.0 * bm * bn * kc / (kCuRate * tile_base(ti) * cu_util(conc));
      if (ns > 1) t += (ns + 1.0) * M * N * 4.0 / kHbm + 3e-6;
      if (t < best_t * 0.999) { best_t = t; best = Plan{ti, ns, kc}; }
    }
  }
  return best;
}

}  // namespace

void gemm(const float* A, const float* B, float* C, int batch, int M, int N, int K, bool transA, bool transB, long sA,
          long sB, long sC, hipStream_t s) {
  if (batch <= 0 || M <= 0 || N <= 0) return;
  if (K <= 0) {  // empty inner dimension: all-zero result (metal.rs:837-839 falls to the CPU loop)
    fill(C, 0.0f, (size_t)batch * M * N, s);
    return;
  }
  if (batch > 65535) fail("malus: gemm batch %d exceeds 65535", batch);
  // float4 staging needs the contiguous dim of each operand to be a multiple of 4
  const bool va = transA ? (M % 4 == 0) : (K % 4 == 0);
  const bool vb = transB ? (K % 4 == 0) : (N % 4 == 0);
  const Plan p = plan_gemm(batch, M, N, K, transA, transB, va, vb);
  static const bool trace = getenv("MALUS_GEMM_TRACE") != nullptr;
  if (trace)
    fprintf(stderr, "malus gemm b%d %dx%dx%d t%d%d -> tile %dx%d occ %d split %d k_chunk %d\n", batch, M, N, K, transA,
            transB, 64 * kTiles[p.ti].tm, 64 * kTiles[p.ti].tn, occupancy(p.ti, transA, transB, va, vb), p.nsplit,
            p.k_chunk);
  const int bm = 64 * kTiles[p.ti].tm, bn = 64 * kTiles[p.ti].tn;
  const int tiles_m = (M + bm - 1) / bm, tiles_n = (N + bn - 1) / bn;
  const int tiles = tiles_m * tiles_n;
  int nsplit = p.nsplit, k_chunk = p.k_chunk;
  const size_t mn = (size_t)M * N;
  size_t bucket = 0;
  float* dst = C;
  if (nsplit > 1) dst = static_cast<float*>(pool_alloc(mn * nsplit * sizeof(float), &bucket));
  long split_stride = nsplit > 1 ? (long)mn : 0;
  void* args[] = {&A, &B, &dst, &M, &N, &K, &sA, &sB, &sC, &k_chunk, const_cast<int*>(&tiles_n), &split_stride};
  MALUS_HIP(hipLaunchKernel(kernel_for(p.ti, transA, transB, va, vb), dim3((unsigned)tiles, (unsigned)nsplit, (unsigned)batch),
                            dim3(256), args, 0, s));
  if (nsplit > 1) {
    size_t blocks = (mn + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    k_split_reduce<<<(unsigned)blocks, 256, 0, s>>>(dst, C, mn, nsplit);
    MALUS_HIP(hipGetLastError());
    pool_free(dst, bucket);
  }
}

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

// Tuning knob: the number of workgroups a split-K GEMM aims for (0 restores
// the cost model's choice).
extern "C" void malus_gemm_set_split(int target_blocks) {
  malus::k::g_split_target = target_blocks > 0 ? target_blocks : 0;
}
