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

#include "common.h"
#include "k_gelu.h"

namespace malus {
namespace k {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int BK = 16;

// The MFMA work of one 16-deep K step from each lane's 8 fragment values
// (k = 8h + s for lane half h, the same k slots in A and B): eight FP32
// 32x32x2 steps, or under autocast (BF) one 32x32x16 bf16 MFMA over the same
// 16 k values, with both operands rounded to bf16 (round to nearest even,
// v_cvt_pk_bf16_f32).  A bf16 product is exact in f32, so BF differs from
// the f32 product only in the operands' rounding and the order of the f32
// accumulation.
template <int TM, int TN, bool BF>
__device__ __forceinline__ void mfma_kstep(const float (&fa)[TM][8], const float (&fb)[TN][8], v16f (&acc)[TM][TN]) {
  if constexpr (BF) {
    bf16x8 a[TM], b[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int e = 0; e < 8; ++e) a[i][e] = (__bf16)fa[i][e];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) b[j][e] = (__bf16)fb[j][e];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
  } else {
#pragma unroll
    for (int st = 0; st < 8; ++st)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fa[i][st], fb[j][st], acc[i][j], 0, 0, 0);
  }
}

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

// ---- LDS-DMA path --------------------------------------------------------------
// When K is a multiple of 16 (and the x-contiguous operands' rows are
// 16-byte multiples), operand slabs move global -> LDS with
// buffer_load_dwordx4 ... lds: no VGPR staging and no LDS store
// instructions.  Lane l of such a wave instruction writes LDS bytes
// [16 l, 16 l + 16) past the wave's base (M0), so each instruction fills a
// dense 1 KB run; the runtime picks which global 16-byte chunk each lane
// fetches.  Layouts (dense, no padding):
//   KC slab: [BX rows][16 k], chunk c of row r stored at chunk c ^ ((r >> 1) & 3)
//            (the swizzle makes the two 128-bit fragment reads per lane
//            bank-conflict-free);
//   XC slab: [16 k][BX] (a half-wave reads 32 consecutive floats).
// Buffer loads past the descriptor's byte count return 0; other reads past a
// matrix edge only feed output rows/columns that are never stored.
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) const float lds_float;
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));

#if defined(__HIP_DEVICE_COMPILE__)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const float* p, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p), (short)0, (int)bytes, 0x00020000);
}
#endif

// Element x of an index map (strides in floats); see GemmMap.  MAP = false
// instances serve dense operands, whose maps are all x * s0.
template <bool MAP>
__device__ __forceinline__ int map_at(const GemmMap& f, int x) {
  if (!MAP) return x * f.s0;
  return f.div ? (x / f.div) * f.s1 + (x % f.div) * f.s0 : x * f.s0;
}

// Byte offset of k row/column k along a k map, advanced one 16-deep slab at
// a time without a division (the host keeps div a multiple of 16).
template <bool MAP>
struct KCursor {
  int q, r;  // k = q * div + r  (r = k for dense maps)
  __device__ __forceinline__ void init(const GemmMap& f, int k) {
    if (MAP && f.div) { q = k / f.div; r = k % f.div; } else { q = 0; r = k; }
  }
  __device__ __forceinline__ int bytes(const GemmMap& f) const { return 4 * ((MAP && f.div) ? q * f.s1 + r * f.s0 : r * f.s0); }
  __device__ __forceinline__ void advance(const GemmMap& f) {
    r += BK;
    if (MAP && f.div && r == f.div) { r = 0; ++q; }
  }
};

// s_waitcnt with vmcnt = N and no wait on the other counters (gfx9
// encoding: vmcnt bits [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8])
template <int N>
__device__ __forceinline__ void waitcnt_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <int BX, bool KC>
struct DmaSlab {
  static constexpr int SIZE = BX * BK;        // floats
  static constexpr int PER_WAVE = SIZE / 1024;  // 1 KB instructions per wave (4 waves)
  static constexpr int READS = KC ? 2 : 4;    // LDS read instructions of one 32-row fragment
  int off[PER_WAVE];                          // byte offset of this lane's chunk at k0 = 0

  // x0: first row/column of the tile.  fx maps the operand's free index x
  // (m for A, n for B), fk its k index; the host guarantees that 4
  // consecutive values of the contiguous index and 16 consecutive k never
  // straddle a map's div (so one slab's k rows sit at fk(k0) + r * fk.s0).
  template <bool MAP>
  __device__ __forceinline__ void init(int x0, const GemmMap& fx, const GemmMap& fk, int wave, int lane) {
#pragma unroll
    for (int q = 0; q < PER_WAVE; ++q) {
      const int c = q * 4 + wave;  // 256-float run of the slab
      if (KC) {
        const int r = c * 16 + lane / 4;
        const int chunk = (lane & 3) ^ ((r >> 1) & 3);
        off[q] = (map_at<MAP>(fx, x0 + r) + 4 * chunk) * 4;
      } else {
        const int f = c * 256 + 4 * lane;
        off[q] = (map_at<MAP>(fx, x0 + f % BX) + (f / BX) * fk.s0) * 4;
      }
    }
  }
#if defined(__HIP_DEVICE_COMPILE__)
  // dk: byte offset of k row/column k0 (fk(k0) * 4), uniform over the block
  __device__ __forceinline__ void issue(__amdgpu_buffer_rsrc_t rs, float* S, int wave, int dk) const {
#pragma unroll
    for (int q = 0; q < PER_WAVE; ++q)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(S + (q * 4 + wave) * 256), 16, off[q] + dk, 0, 0, 0);
  }
#endif
  // The 8 MFMA-step values (k = 8h .. 8h + 7) of lane (i, h) for tile rows xw ..
  // The reads are inline asm: the compiler treats any LDS read after an
  // LDS-DMA load as a possible alias of it and would wait for every DMA in
  // flight, including the slabs prefetched into other stages.  The caller
  // waits (lgkmcnt) before the values are used.
  __device__ __forceinline__ static void frag(const float* __restrict__ S, int xw, float f[8]) {
#if defined(__HIP_DEVICE_COMPILE__)
    const int lane = threadIdx.x & 63, i = lane & 31, h = lane >> 5;
    const unsigned base = (unsigned)(uintptr_t)(const lds_float*)S;
    if (KC) {
      const int r = xw + i, sw = (r >> 1) & 3;
      v4f a, b;
      asm volatile("ds_read_b128 %0, %1" : "=v"(a) : "v"(base + 4u * (r * BK + 4 * ((2 * h) ^ sw))));
      asm volatile("ds_read_b128 %0, %1" : "=v"(b) : "v"(base + 4u * (r * BK + 4 * ((2 * h + 1) ^ sw))));
      f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
      f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    } else {
      // rows 8h + s, s = 0..7, are BX floats apart: pairs via the 64-dword stride form
      static_assert(BX % 64 == 0, "x-contiguous slab rows are whole 64-dword strides");
      constexpr int ST = BX / 64;
      const unsigned a0 = base + 4u * (8 * h * BX + xw + i);
      v2f p0, p1, p2, p3;
      asm volatile("ds_read2st64_b32 %0, %1 offset1:%2" : "=v"(p0) : "v"(a0), "i"(ST));
      asm volatile("ds_read2st64_b32 %0, %1 offset0:%2 offset1:%3" : "=v"(p1) : "v"(a0), "i"(2 * ST), "i"(3 * ST));
      asm volatile("ds_read2st64_b32 %0, %1 offset0:%2 offset1:%3" : "=v"(p2) : "v"(a0), "i"(4 * ST), "i"(5 * ST));
      asm volatile("ds_read2st64_b32 %0, %1 offset0:%2 offset1:%3" : "=v"(p3) : "v"(a0), "i"(6 * ST), "i"(7 * ST));
      f[0] = p0.x; f[1] = p0.y; f[2] = p1.x; f[3] = p1.y;
      f[4] = p2.x; f[5] = p2.y; f[6] = p3.x; f[7] = p3.y;
    }
#endif
  }
};

// Same contract as k_sgemm, with each operand addressed through its
// GemmLayout (batch, row and column maps of the stored matrix; C's also
// addresses D).  Dense row-major operands are the maps {0, 0, ld}.  The
// host guarantees K % 16 == 0, the map conditions above, and every byte
// offset below 2^31; a split-K launch writes dense partials.
// EPI: 0 plain; 1 also E = gelu(C) (the GELU after a GEMM, no D); 2 C =
// gelu_bwd(E, product) (+ D): the GELU VJP applied to the product, with E
// the GELU input; 3 accumulate L.ngroup products in group order,
// C = ((D + A0 op B0) + A1 op B1) + ..., each product rounded to f32 before
// its add (the rounding of one GEMM per group with its addend chained).
// E shares C's layout.  Grouped launches (L.ngroup > 1, MAP only): with
// EPI != 3, workgroup z runs group z (its own A, B, C); the batch index is 0.
template <int TM, int TN, bool TA, bool TB, bool MAP, int EPI = 0, bool BF = false>
__global__ __launch_bounds__(256, 2) void k_sgemm_dma(const float* __restrict__ A, const float* __restrict__ B,
                                                      float* __restrict__ C, int M, int N, int K, GemmLayouts L,
                                                      int k_chunk, int tiles_n, long split_stride,
                                                      const float* __restrict__ D, float* __restrict__ E) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int BM = 64 * TM, BN = 64 * TN;
  using SlabA = DmaSlab<BM, !TA>;  // A [M][K] is k-contiguous
  using SlabB = DmaSlab<BN, TB>;   // B^T [N][K] is k-contiguous
  // Two-stage ring of KS 16-deep slabs per stage: stage st + 1 is in
  // flight while stage st is consumed.  Under autocast (BF) a slab's MFMA
  // work is one bf16 instruction per accumulator, so the barrier and the
  // fragment reads dominate; two slabs per stage halve the barriers and let
  // the second slab's reads overlap the first slab's MFMAs (f32 K steps are
  // long enough that one slab per stage measured faster).
  // (Three- and four-stage rings measured no faster for either precision.)
  constexpr bool BFS = BF && (BM + BN <= 256);
  constexpr int NS = 2, KS = BFS ? 2 : 1;
  constexpr int PER_SLAB = SlabA::PER_WAVE + SlabB::PER_WAVE;  // DMA instructions per slab and wave
  // LDS reads of one slab's fragments (lgkmcnt is 4 bits)
  constexpr int READS = TM * SlabA::READS + TN * SlabB::READS;
  __shared__ __attribute__((aligned(1024))) float As[NS][KS][SlabA::SIZE];
  __shared__ __attribute__((aligned(1024))) float Bs[NS][KS][SlabB::SIZE];

  // Workgroups are dealt to the 8 XCDs round-robin in dispatch order (x
  // fastest, then y), and each XCD has its own L2.  Tile ids are remapped so
  // that every XCD gets a contiguous range of the work: consecutive tiles of
  // one output row without a K split; with one (the weight gradients, K =
  // tokens), a contiguous range of the split-major list, so an XCD's
  // workgroups share one k range of both operands instead of every XCD
  // reading the whole K range of some output columns (3x fewer HBM bytes
  // on the C5 weight gradients).
  const int nt = gridDim.x, ns = gridDim.y;
  int tile, split;
  if (ns == 1) {
    tile = blockIdx.x;
    if ((nt & 7) == 0) tile = (tile & 7) * (nt >> 3) + (tile >> 3);
    split = 0;
  } else {
    const int total = nt * ns, lin = blockIdx.x + nt * blockIdx.y;
    const int w = (total & 7) == 0 ? (lin & 7) * (total >> 3) + (lin >> 3) : lin;
    split = w / nt;
    tile = w % nt;
  }
  const int tm = tile / tiles_n, tn = tile % tiles_n;
  const int m0 = tm * BM, n0 = tn * BN;
  const bool grouped = MAP && L.ngroup > 1;
  const int b = grouped ? 0 : blockIdx.z;
  if (grouped && EPI != 3) {
    A = L.ga[blockIdx.z];
    B = L.gb[blockIdx.z];
    C = L.gc[blockIdx.z];
  }
  const int ba = map_at<MAP>(L.a.b, b), bb = map_at<MAP>(L.b.b, b);
  C += map_at<MAP>(L.c.b, b) + (long)split * split_stride;
  if (D) D += map_at<MAP>(L.c.b, b);
  if (EPI == 1 || EPI == 2) E += map_at<MAP>(L.c.b, b);
  int kbeg = split * k_chunk;
  int kend = min(K, kbeg + k_chunk);
  if (MAP && L.tri_a) {  // op(A) row m is zero past k = m (A) or before k = m (A^T stored lower-triangular)
    if (TA) kbeg = max(kbeg, m0);
    else kend = min(kend, m0 + BM);
  }

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = (wave >> 1) * 32 * TM, wn = (wave & 1) * 32 * TN;
  const int li = lane & 31, lk = lane >> 5;
  // stored A: [M][K] (rows m) or [K][M] (rows k); stored B: [K][N] or [N][K]
  const GemmMap& fam = TA ? L.a.c : L.a.r;
  const GemmMap& fak = TA ? L.a.r : L.a.c;
  const GemmMap& fbn = TB ? L.b.r : L.b.c;
  const GemmMap& fbk = TB ? L.b.c : L.b.r;
  SlabA sa;
  SlabB sb;
  sa.template init<MAP>(m0, fam, fak, wave, lane);
  sb.template init<MAP>(n0, fbn, fbk, wave, lane);

  v16f acc[TM][TN];
  const int nk = kend > kbeg ? (kend - kbeg) / BK : 0;
  // acc = op(A) @ op(B) over [kbeg, kend) for operands Ap, Bp
  auto run_k = [&](const float* Ap, const float* Bp) {
    const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(Ap + ba, (unsigned)((L.ext_a - ba) * 4));
    const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(Bp + bb, (unsigned)((L.ext_b - bb) * 4));
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = v16f{0};
    KCursor<MAP> ka, kb;
    ka.init(fak, kbeg);
    kb.init(fbk, kbeg);
    const int nst = (nk + KS - 1) / KS;
    auto issue_stage = [&](int st, int buf) {
#pragma unroll
      for (int u = 0; u < KS; ++u)
        if (st * KS + u < nk) {
          sa.issue(ra, As[buf][u], wave, ka.bytes(fak));
          sb.issue(rb, Bs[buf][u], wave, kb.bytes(fbk));
          ka.advance(fak);
          kb.advance(fbk);
        }
    };
#pragma unroll
    for (int p = 0; p < NS - 1; ++p)
      if (p < nst) issue_stage(p, p);
    int cur = 0;
    for (int st = 0; st < nst; ++st) {
      // stage st has landed once at most the NS - 2 full stages issued after
      // it are in flight (this wave's loads complete in order); the barrier
      // makes every wave's part visible and retires the reads of stage st - 1
      if (st + NS - 2 < nst - 1) waitcnt_vm<(NS - 2) * KS * PER_SLAB>();
      else waitcnt_vm<0>();
      __builtin_amdgcn_s_barrier();
      const bool two = KS == 2 && st * KS + 1 < nk;
      float fa[KS][TM][8], fb[KS][TN][8];
#pragma unroll
      for (int i = 0; i < TM; ++i) SlabA::frag(As[cur][0], wm + 32 * i, fa[0][i]);
#pragma unroll
      for (int j = 0; j < TN; ++j) SlabB::frag(Bs[cur][0], wn + 32 * j, fb[0][j]);
      __builtin_amdgcn_sched_barrier(0);
      // stage st - 1 (= st + NS - 1 mod NS) was last read before the barrier
      const int nxt = cur == 0 ? NS - 1 : cur - 1;
      if (st + NS - 1 < nst) issue_stage(st + NS - 1, nxt);
      if constexpr (KS == 2) {
        // The second slab's fragments are read on every path, also in a last
        // stage that holds one slab (an odd slab count; the values then go
        // unused), so the waits below do not depend on a branch.
#pragma unroll
        for (int i = 0; i < TM; ++i) SlabA::frag(As[cur][KS - 1], wm + 32 * i, fa[KS - 1][i]);
#pragma unroll
        for (int j = 0; j < TN; ++j) SlabB::frag(Bs[cur][KS - 1], wn + 32 * j, fb[KS - 1][j]);
        // LDS reads complete in order: the first slab's are done when at
        // most the second slab's READS are outstanding
        if constexpr (READS <= 15) asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(READS) : "memory");
        else asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      } else {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the fragment reads above
      }
      __builtin_amdgcn_sched_barrier(0);
      // a wave with MFMAs to issue goes ahead of the CU's other waves (measured
      // 1 % on the C5 step; raising it from the barrier on instead lost 2 %)
      __builtin_amdgcn_s_setprio(1);
      mfma_kstep<TM, TN, BF>(fa[0], fb[0], acc);
      __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (KS == 2) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        if (two) {
          __builtin_amdgcn_s_setprio(1);
          mfma_kstep<TM, TN, BF>(fa[KS - 1], fb[KS - 1], acc);
          __builtin_amdgcn_s_setprio(0);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      cur = cur == NS - 1 ? 0 : cur + 1;
    }
    __syncthreads();  // every wave is done with the stages before they are reused
  };

  // Element (i, j, r) of the wave's accumulators is C at offset
  // cn(i, j) + dm(r) * row stride; C rows come in aligned 32-row groups (the
  // host keeps the row map's div a multiple of 32), so one map evaluation
  // per group and per column.
  auto for_each = [&](auto&& f) {
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int rbase = map_at<MAP>(L.c.r, m0 + wm + 32 * i);
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = n0 + wn + 32 * j + li;
        const int cn = map_at<MAP>(L.c.c, n) + rbase;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dm = 8 * (r >> 2) + 4 * lk + (r & 3);
          const int m = m0 + wm + 32 * i + dm;
          f(i, j, r, n < N && m < M, cn + dm * L.c.r.s0);
        }
      }
    }
  };

  // The epilogue's operand read (the addend D, or E for the GELU VJP) is
  // issued before the K loop, so its latency hides under the MFMAs instead
  // of stalling every workgroup's epilogue at once.  Small wave tiles only:
  // it holds another TM * TN * 16 registers, so only instances that read
  // one (the dense GEMMs that take an addend, the GELU VJP, the grouped
  // accumulation) carry it.  Without it (4 -> 6 workgroups per CU on the
  // 128x64 tiles) the C5 step measured 0.7 % slower for the GELU VJP alone
  // and 1.7 % slower for the dense forms.
  constexpr bool PF = TM * TN <= 2 && ((EPI == 0 && !MAP) || EPI == 2 || EPI == 3);
  const float* pre_src = EPI == 2 ? E : D;
  v16f pre[PF ? TM : 1][PF ? TN : 1];
  if (PF && pre_src)
    for_each([&](int i, int j, int r, bool live, int o) {
      if (PF) pre[i][j][r] = live ? pre_src[o] : 0.0f;
    });
  auto pre_at = [&](int i, int j, int r, int o) -> float {
    if constexpr (PF) return pre[i][j][r];
    else return pre_src[o];
  };

  if constexpr (EPI == 3) {
    v16f tot[TM][TN];
    for (int g = 0; g < L.ngroup; ++g) {
      run_k(L.ga[g], L.gb[g]);
      if (g == 0) {
        for_each([&](int i, int j, int r, bool live, int o) {
          tot[i][j][r] = D && live ? pre_at(i, j, r, o) + acc[i][j][r] : acc[i][j][r];
        });
      } else {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) tot[i][j][r] = tot[i][j][r] + acc[i][j][r];
      }
    }
    for_each([&](int i, int j, int r, bool live, int o) {
      if (live) C[o] = tot[i][j][r];
    });
  } else {
    run_k(A, B);
    for_each([&](int i, int j, int r, bool live, int o) {
      if (live) {
        float v = acc[i][j][r];
        if (EPI == 2) v = gelu_bwd(pre_at(i, j, r, o), v);
        C[o] = D ? (EPI == 2 ? D[o] : pre_at(i, j, r, o)) + v : v;
        if (EPI == 1) E[o] = gelu_fwd(v);
      }
    });
  }
#endif
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

// Variant code: bit 8 = bf16 MFMA (autocast), bit 7 = grouped accumulation,
// bit 6 = GELU epilogues, bit 5 = mapped operands, bit 4 = LDS-DMA path,
// bits 3..0 = transA, transB, vecA, vecB.
constexpr int kVarBf16 = 256;
inline int variant(bool ta, bool tb, bool va, bool vb, bool dma) {
  return (dma << 4) | (ta << 3) | (tb << 2) | (va << 1) | (int)vb;
}

template <int TM, int TN, bool TA, bool TB, bool BF>
const void* kernel_of(int v) {
  if (v & 128) {  // grouped accumulation: mapped NT (the head projections' dA)
    if constexpr (!TA && TB) return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, false, true, true, 3, BF>);
    return nullptr;
  }
  if (v & 64) {  // GELU epilogues: dense NN (forward) and NT (the VJP's dA)
    if constexpr (!TA && !TB) return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, false, false, false, 1, BF>);
    if constexpr (!TA && TB) return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, false, true, false, 2, BF>);
    return nullptr;
  }
  if (v & 32) return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, TA, TB, true, 0, BF>);
  if (v & 16) return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, TA, TB, false, 0, BF>);
  const bool va = v & 2, vb = v & 1;
  if (va && vb) return reinterpret_cast<const void*>(&k_sgemm<TM, TN, TA, TB, true, true, BF>);
  if (va) return reinterpret_cast<const void*>(&k_sgemm<TM, TN, TA, TB, true, false, BF>);
  if (vb) return reinterpret_cast<const void*>(&k_sgemm<TM, TN, TA, TB, false, true, BF>);
  return reinterpret_cast<const void*>(&k_sgemm<TM, TN, TA, TB, false, false, BF>);
}

template <int TM, int TN, bool BF>
const void* kernel_of_layout(int v) {
  const bool ta = v & 8, tb = v & 4;
  if (!ta && !tb) return kernel_of<TM, TN, false, false, BF>(v);
  if (!ta && tb) return kernel_of<TM, TN, false, true, BF>(v);
  if (ta && !tb) return kernel_of<TM, TN, true, false, BF>(v);
  return kernel_of<TM, TN, true, true, BF>(v);
}

template <bool BF>
const void* kernel_for_prec(int ti, int v) {
  switch (ti) {
    case 0: return kernel_of_layout<2, 3, BF>(v);
    case 1: return kernel_of_layout<2, 2, BF>(v);
    case 2: return kernel_of_layout<2, 1, BF>(v);
    case 3: return kernel_of_layout<1, 2, BF>(v);
    default: return kernel_of_layout<1, 1, BF>(v);
  }
}

const void* kernel_for(int ti, int v) {
  return (v & kVarBf16) ? kernel_for_prec<true>(ti, v) : kernel_for_prec<false>(ti, v);
}

// Co-resident workgroups per CU of each kernel variant (VGPR and LDS
// limited), from the runtime's occupancy calculator; cached per variant.
int occupancy(int ti, int v) {
  static int cache[kNumTiles][512];
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

// Pick the tile and the K split with the smallest modelled time: the
// busiest CU's MFMA work (256 CUs at 75 % of 157.3 TFLOP/s, scaled by the
// tile's efficiency and the CU's concurrency), plus the split-K partials'
// HBM round trip.  Long-K shapes with few output tiles (the weight-gradient
// GEMMs, K = tokens) split K so the grid fills the chip's workgroup slots.
// tri: A lower-triangular (GemmLayouts::tri_a); a tile row then runs on
// average (n + 1) / (2 n) of K for n tile rows, which favours short tiles.
Plan plan_gemm(int batch, int M, int N, int K, int v, bool tri = false, int only_tile = -1) {
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
  const bool wgrad_bf = wgrad && g_autocast;
  if (wgrad_bf) only_tile = 0;  // kTiles[0] = 128x192
  for (int ti = 0; ti < kNumTiles; ++ti) {
    if (g_forced_tile >= 0 && ti != g_forced_tile) continue;
    if (only_tile >= 0 && g_forced_tile < 0 && ti != only_tile) continue;
    const int bm = 64 * kTiles[ti].tm, bn = 64 * kTiles[ti].tn;
    if (wgrad && !wgrad_bf &&
        !((kTiles[ti].tm == 2 && kTiles[ti].tn == 1) || (kTiles[ti].tm == 1 && kTiles[ti].tn == 2)))
      continue;
    const long tiles = (long)((M + bm - 1) / bm) * ((N + bn - 1) / bn) * batch;
    const int occ = occupancy(ti, v);
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
  // mapped GEMM splits K exactly like its dense twin
  const int v = variant(transA, transB, false, false, true);
  // Under autocast the GELU GEMM (h = x W1, K = 384, a 3072-workgroup grid
  // at 128x64) measured 20 % faster on 128x192 tiles.
  Plan p = plan_gemm(batch, M, N, K, v, mapped && L.tri_a, g_autocast && epi == 1 ? 0 : -1);
  const char* tag = mapped ? " mapped" : "";
  if ((!split_ok || epi) && p.nsplit > 1) {
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
  const int vb = (epi ? v | 64 : mapped ? v | 32 : v) | (g_autocast ? kVarBf16 : 0);
  const void* fn = kernel_for(p.ti, vb);
  if (!fn) fail("malus: gemm: no kernel for epilogue %d with transA=%d transB=%d", epi, transA, transB);
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

bool map_contig4(const GemmMap& f) { return f.s0 == 1 && (f.div == 0 || f.div % 4 == 0); }
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
          long sB, long sC, hipStream_t s, const float* D) {
  if (batch <= 0 || M <= 0 || N <= 0) return;
  if (K <= 0) {  // empty inner dimension: all-zero result (metal.rs:837-839 falls to the CPU loop)
    fill(C, 0.0f, (size_t)batch * M * N, s);
    return;
  }
  if (batch > 65535) fail("malus: gemm batch %d exceeds 65535", batch);
  const long lda = transA ? M : K, ldb = transB ? K : N;
  const long ext_a = (long)(batch - 1) * sA + (long)M * K, ext_b = (long)(batch - 1) * sB + (long)K * N;
  // LDS-DMA path: whole 16-deep K slabs, 16-byte rows, 32-bit byte offsets
  const bool dma = K % 16 == 0 && (transA ? M % 4 == 0 : true) && (transB ? true : N % 4 == 0) &&
                   (size_t)ext_a * 4 < (1ull << 31) && (size_t)ext_b * 4 < (1ull << 31) &&
                   ((size_t)(batch - 1) * sC + (size_t)M * N) * 4 < (1ull << 31) && g_allow_dma;
  if (dma) {
    GemmLayouts L{dense_layout(lda, sA), dense_layout(ldb, sB), dense_layout(N, sC), (int)ext_a, (int)ext_b};
    launch_dma(A, B, C, batch, M, N, K, transA, transB, L, s, D, true, false);
    return;
  }
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
               hipStream_t s, const float* D) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 16 || N % 4 || !g_allow_dma || (!backward && (D || transB)) ||
      (backward && !transB))
    return false;
  const long ext_a = (long)M * K, ext_b = (long)K * N;
  if ((size_t)ext_a * 4 >= (1ull << 31) || (size_t)ext_b * 4 >= (1ull << 31) || (size_t)M * N * 4 >= (1ull << 31))
    return false;
  GemmLayouts L{dense_layout(K, 0), dense_layout(transB ? K : N, 0), dense_layout(N, 0), (int)ext_a, (int)ext_b};
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
  Plan p = plan_gemm(1, M, N, K, v);
  const bool c_dense = L.c.r.div == 0 && L.c.c.div == 0 && L.c.c.s0 == 1 && L.c.r.s0 == N;
  if (accumulate || !c_dense) {
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
  const void* fn = kernel_for(p.ti, (accumulate ? v | 128 : v | 32) | (g_autocast ? kVarBf16 : 0));
  if (!fn) fail("malus: gemm_grouped: no kernel for transA=%d transB=%d", transA, transB);
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
  // contiguous dimension of each stored operand: runs of 4 floats
  const GemmMap& a_contig = L.a.c;  // A [M][K]: k;  A^T [K][M]: m
  const GemmMap& b_contig = L.b.c;  // B [K][N]: n;  B^T [N][K]: k
  if (!map_contig4(a_contig) || !map_contig4(b_contig)) return false;
  if (transA ? M % 4 : 0) return false;
  if (transB ? 0 : N % 4) return false;
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

// Tuning knob: 0 keeps every GEMM on the register-staged path (for A/B
// comparisons); 1 (default) uses the LDS-DMA path where the shape allows.
extern "C" void malus_gemm_set_dma(int on) { malus::k::g_allow_dma = on != 0; }

// Tuning knob: the number of workgroups a split-K GEMM aims for (0 restores
// the cost model's choice).
extern "C" void malus_gemm_set_split(int target_blocks) {
  malus::k::g_split_target = target_blocks > 0 ? target_blocks : 0;
}
