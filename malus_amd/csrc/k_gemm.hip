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
// Tiling: 256 threads (4 waves in a 2x2 grid), block tile 128x128, BK = 16,
// each wave owns a 64x64 sub-tile = 2x2 MFMA 32x32 accumulators (64 fp32
// accumulator registers per lane).  Operand tiles are staged in LDS as
// [k][m] / [k][n] so every MFMA operand read is 32 consecutive floats per
// half-wave; global->LDS staging is double-buffered with one barrier per
// K step.  Long-K shapes with few output tiles (the weight-gradient GEMMs,
// K = tokens) split K across workgroups and reduce the partials in split
// order, which keeps results deterministic.  Tile ids are remapped so
// consecutive tiles of one output row land on the same XCD (shared L2).
//
// MFMA lane layout (verified on gfx950): A[i][k] from lane i + 32k,
// B[k][j] from lane j + 32k, D register r of lane l holds
// D[8*(r/4) + 4*(l/32) + r%4][l%32].
#include "common.h"

namespace malus {
namespace k {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 16, PAD = 4;
constexpr int LDA_S = BM + PAD, LDB_S = BN + PAD;

template <bool TA, bool VA>
struct ALoader {
  float r[8];
  // Load the BMxBK tile starting at (m0, k0) into registers.  K is the row
  // stride of a row-major A ([M][K]); k indices >= klim read as zero.
  __device__ __forceinline__ void load(const float* __restrict__ A, int M, int K, int klim, int m0, int k0) {
    const int t = threadIdx.x;
    if (VA) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        int idx = t + 256 * q;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (!TA) {
          int rr = idx >> 2, c4 = idx & 3;
          int m = m0 + rr, k = k0 + c4 * 4;
          if (m < M && k < klim) v = *reinterpret_cast<const float4*>(A + (size_t)m * K + k);
        } else {
          int kr = idx >> 5, c4 = idx & 31;
          int k = k0 + kr, m = m0 + c4 * 4;
          if (k < klim && m < M) v = *reinterpret_cast<const float4*>(A + (size_t)k * M + m);
        }
        r[4 * q] = v.x; r[4 * q + 1] = v.y; r[4 * q + 2] = v.z; r[4 * q + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        int e = t + 256 * q;
        float v = 0.f;
        if (!TA) {
          int rr = e >> 4, kk = e & 15;
          int m = m0 + rr, k = k0 + kk;
          if (m < M && k < klim) v = A[(size_t)m * K + k];
        } else {
          int kr = e >> 7, mm = e & 127;
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
      for (int q = 0; q < 2; ++q) {
        int idx = t + 256 * q;
        if (!TA) {
          int rr = idx >> 2, c4 = idx & 3;
#pragma unroll
          for (int j = 0; j < 4; ++j) As[(c4 * 4 + j) * LDA_S + rr] = r[4 * q + j];
        } else {
          int kr = idx >> 5, c4 = idx & 31;
          *reinterpret_cast<float4*>(As + kr * LDA_S + c4 * 4) = make_float4(r[4 * q], r[4 * q + 1], r[4 * q + 2], r[4 * q + 3]);
        }
      }
    } else {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        int e = t + 256 * q;
        if (!TA) As[(e & 15) * LDA_S + (e >> 4)] = r[q];
        else As[(e >> 7) * LDA_S + (e & 127)] = r[q];
      }
    }
  }
};

template <bool TB, bool VB>
struct BLoader {
  float r[8];
  // K is the row stride of a transposed B ([N][K]); k >= klim reads zero.
  __device__ __forceinline__ void load(const float* __restrict__ B, int N, int K, int klim, int n0, int k0) {
    const int t = threadIdx.x;
    if (VB) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        int idx = t + 256 * q;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (!TB) {
          int kr = idx >> 5, c4 = idx & 31;
          int k = k0 + kr, n = n0 + c4 * 4;
          if (k < klim && n < N) v = *reinterpret_cast<const float4*>(B + (size_t)k * N + n);
        } else {
          int rr = idx >> 2, c4 = idx & 3;
          int n = n0 + rr, k = k0 + c4 * 4;
          if (n < N && k < klim) v = *reinterpret_cast<const float4*>(B + (size_t)n * K + k);
        }
        r[4 * q] = v.x; r[4 * q + 1] = v.y; r[4 * q + 2] = v.z; r[4 * q + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        int e = t + 256 * q;
        float v = 0.f;
        if (!TB) {
          int kr = e >> 7, nn = e & 127;
          int k = k0 + kr, n = n0 + nn;
          if (k < klim && n < N) v = B[(size_t)k * N + n];
        } else {
          int rr = e >> 4, kk = e & 15;
          int n = n0 + rr, k = k0 + kk;
          if (n < N && k < klim) v = B[(size_t)n * K + k];
        }
        r[q] = v;
      }
    }
  }
  __device__ __forceinline__ void store(float* __restrict__ Bs) const {
    const int t = threadIdx.x;
    if (VB) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        int idx = t + 256 * q;
        if (!TB) {
          int kr = idx >> 5, c4 = idx & 31;
          *reinterpret_cast<float4*>(Bs + kr * LDB_S + c4 * 4) = make_float4(r[4 * q], r[4 * q + 1], r[4 * q + 2], r[4 * q + 3]);
        } else {
          int rr = idx >> 2, c4 = idx & 3;
#pragma unroll
          for (int j = 0; j < 4; ++j) Bs[(c4 * 4 + j) * LDB_S + rr] = r[4 * q + j];
        }
      }
    } else {
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        int e = t + 256 * q;
        if (!TB) Bs[(e >> 7) * LDB_S + (e & 127)] = r[q];
        else Bs[(e & 15) * LDB_S + (e >> 4)] = r[q];
      }
    }
  }
};

// grid: x = output tiles (XCD-remapped), y = K splits, z = batch.
// Split s writes its partial tile to C + s * split_stride (split_stride = 0
// when there is one split).
template <bool TA, bool TB, bool VA, bool VB>
__global__ __launch_bounds__(256, 2) void k_sgemm(const float* __restrict__ A, const float* __restrict__ B,
                                                  float* __restrict__ C, int M, int N, int K, long sA, long sB, long sC,
                                                  int k_chunk, int tiles_n, long split_stride) {
  __shared__ __attribute__((aligned(16))) float As[2][BK * LDA_S];
  __shared__ __attribute__((aligned(16))) float Bs[2][BK * LDB_S];

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
  const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
  const int li = lane & 31, lk = lane >> 5;

  v16f acc00 = {0}, acc01 = {0}, acc10 = {0}, acc11 = {0};

  ALoader<TA, VA> la;
  BLoader<TB, VB> lb;
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
    const float* as = As[cur];
    const float* bs = Bs[cur];
#pragma unroll
    for (int kk = 0; kk < BK / 2; ++kk) {
      const int kr = 2 * kk + lk;
      float a0 = as[kr * LDA_S + wm + li];
      float a1 = as[kr * LDA_S + wm + 32 + li];
      float b0 = bs[kr * LDB_S + wn + li];
      float b1 = bs[kr * LDB_S + wn + 32 + li];
      acc00 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b0, acc00, 0, 0, 0);
      acc01 = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, b1, acc01, 0, 0, 0);
      acc10 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b0, acc10, 0, 0, 0);
      acc11 = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, b1, acc11, 0, 0, 0);
    }
    if (more) {
      la.store(As[cur ^ 1]);
      lb.store(Bs[cur ^ 1]);
    }
    __syncthreads();
  }

  // epilogue: D register r of lane l -> row 8*(r/4) + 4*(l/32) + r%4, col l%32
  auto store_tile = [&](const v16f& acc, int ti, int tj) {
    const int n = n0 + wn + tj * 32 + li;
    if (n >= N) return;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int m = m0 + wm + ti * 32 + 8 * (r >> 2) + 4 * lk + (r & 3);
      if (m < M) C[(size_t)m * N + n] = acc[r];
    }
  };
  store_tile(acc00, 0, 0);
  store_tile(acc01, 0, 1);
  store_tile(acc10, 1, 0);
  store_tile(acc11, 1, 1);
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

template <bool TA, bool TB>
void launch_variant(bool va, bool vb, dim3 grid, hipStream_t s, const float* A, const float* B, float* C, int M, int N,
                    int K, long sA, long sB, long sC, int k_chunk, int tiles_n, long split_stride) {
  if (va && vb) k_sgemm<TA, TB, true, true><<<grid, 256, 0, s>>>(A, B, C, M, N, K, sA, sB, sC, k_chunk, tiles_n, split_stride);
  else if (va) k_sgemm<TA, TB, true, false><<<grid, 256, 0, s>>>(A, B, C, M, N, K, sA, sB, sC, k_chunk, tiles_n, split_stride);
  else if (vb) k_sgemm<TA, TB, false, true><<<grid, 256, 0, s>>>(A, B, C, M, N, K, sA, sB, sC, k_chunk, tiles_n, split_stride);
  else k_sgemm<TA, TB, false, false><<<grid, 256, 0, s>>>(A, B, C, M, N, K, sA, sB, sC, k_chunk, tiles_n, split_stride);
}

}  // namespace

void gemm(const float* A, const float* B, float* C, int batch, int M, int N, int K, bool transA, bool transB, long sA,
          long sB, long sC, hipStream_t s) {
  if (batch <= 0 || M <= 0 || N <= 0) return;
  if (K <= 0) {  // empty inner dimension: all-zero result (metal.rs:837-839 falls to the CPU loop)
    fill(C, 0.0f, (size_t)batch * M * N, s);
    return;
  }
  // float4 staging needs the contiguous dim of each operand to be a multiple of 4
  const bool va = transA ? (M % 4 == 0) : (K % 4 == 0);
  const bool vb = transB ? (K % 4 == 0) : (N % 4 == 0);
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int tiles = tiles_m * tiles_n;
  int nsplit = 1;
  if (batch == 1 && tiles < 256 && K >= 1024) {
    nsplit = (512 + tiles - 1) / tiles;
    int max_split = K / 256;
    if (nsplit > max_split) nsplit = max_split;
    if (nsplit < 1) nsplit = 1;
  }
  int k_chunk = (K + nsplit - 1) / nsplit;
  k_chunk = (k_chunk + BK - 1) / BK * BK;
  nsplit = (K + k_chunk - 1) / k_chunk;
  if (batch > 65535) fail("malus: gemm batch %d exceeds 65535", batch);
  dim3 grid((unsigned)tiles, (unsigned)nsplit, (unsigned)batch);
  float* dst = C;
  size_t bucket = 0;
  const size_t mn = (size_t)M * N;
  if (nsplit > 1) dst = static_cast<float*>(pool_alloc(mn * nsplit * sizeof(float), &bucket));
  const long split_stride = nsplit > 1 ? (long)mn : 0;
  if (!transA && !transB) launch_variant<false, false>(va, vb, grid, s, A, B, dst, M, N, K, sA, sB, sC, k_chunk, tiles_n, split_stride);
  else if (!transA && transB) launch_variant<false, true>(va, vb, grid, s, A, B, dst, M, N, K, sA, sB, sC, k_chunk, tiles_n, split_stride);
  else if (transA && !transB) launch_variant<true, false>(va, vb, grid, s, A, B, dst, M, N, K, sA, sB, sC, k_chunk, tiles_n, split_stride);
  else launch_variant<true, true>(va, vb, grid, s, A, B, dst, M, N, K, sA, sB, sC, k_chunk, tiles_n, split_stride);
  MALUS_HIP(hipGetLastError());
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
