// LDS-DMA GEMM kernels for gfx950 (v_mfma_f32_32x32x2_f32, and the bf16
// MFMA under autocast), shared by k_gemm.hip, k_gemm_io.hip and k_gemm_io_w.hip.
#pragma once
#include <type_traits>

#include "common.h"
#include "k_gelu.h"
#include "k_split.h"

namespace malus {
namespace k {

// The LDS-DMA instance for tile index ti (of the host's tile table) and a
// variant whose bits 12..9 carry GemmLayouts::io (k_gemm_io.hip); null for
// the combinations no caller uses.
const void* gemm_io_kernel(int ti, int v);
// The same for the instances with a bf16 weight as B (k_gemm_io_w.hip).
const void* gemm_io_weight_kernel(int ti, int v);
// The same for the split-product instances with a weight's split copy as B
// (kIoB3, k_gemm_io_x3.hip).
const void* gemm_io_x3_kernel(int ti, int v);

namespace {

typedef float v4f_raw __attribute__((ext_vector_type(4)));  // 4 words of packed bf16 pairs

constexpr int BK = 16;

// The MFMA work of one 16-deep K step from each lane's 8 fragment values
// (k = 8h + s for lane half h, the same k slots in A and B): eight FP32
// 32x32x2 steps, or under autocast (BF) one 32x32x16 bf16 MFMA over the same
// 16 k values, with both operands rounded to bf16 (round to nearest even,
// v_cvt_pk_bf16_f32).  A bf16 product is exact in f32, so BF differs from
// the f32 product only in the operands' rounding and the order of the f32
// accumulation.
// A16 / B16: that operand's fragments arrive as bf16 already (operands
// stored in bf16): words 0..3 of its 8 slots hold the 8 bf16 values, k
// order unchanged, so the instruction sees the same values as when an f32
// copy of the rounded operand is rounded here.
// X3: the f32 product on the bf16 MFMA from exact three-way splits of
// both operands (k_split.h), the same slab step the fused attention
// kernels run.
// X3 with B read as its three stored pieces (kIoB3: a weight's split copy):
// fb holds TN fragments of each plane, h first; words 0..3 of a fragment
// hold its 8 bf16 values, as in a bf16-stored operand.  Only A is split.
template <int TM, int TN>
__device__ __forceinline__ void mfma_kstep_b3(const float (&fa)[TM][8], const float (&fb)[3 * TN][8],
                                              v16f (&acc)[TM][TN]) {
  Split3 a[TM], b[TN];
#pragma unroll
  for (int i = 0; i < TM; ++i) a[i] = split3(fa[i]);
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    auto plane = [&](int p) {
      const float(&f)[8] = fb[p * TN + j];
      return __builtin_bit_cast(bf16x8, (v4f_raw){f[0], f[1], f[2], f[3]});
    };
    b[j] = Split3{plane(0), plane(1), plane(2)};
  }
  x3_slab<false, TM, TN>(a, b, acc);
}

template <int TM, int TN, bool BF, bool A16 = false, bool B16 = false, bool X3 = false>
__device__ __forceinline__ void mfma_kstep(const float (&fa)[TM][8], const float (&fb)[TN][8], v16f (&acc)[TM][TN]) {
  static_assert(BF || !(A16 || B16), "bf16-stored operands run on the bf16 MFMA");
  static_assert(!X3 || (BF && !A16 && !B16), "the split product reads f32 operands");
  if constexpr (X3) {
    Split3 a[TM], b[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) a[i] = split3(fa[i]);
#pragma unroll
    for (int j = 0; j < TN; ++j) b[j] = split3(fb[j]);
    x3_slab<false, TM, TN>(a, b, acc);
  } else if constexpr (BF) {
    bf16x8 a[TM], b[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      if constexpr (A16) {
        a[i] = __builtin_bit_cast(bf16x8, (v4f_raw){fa[i][0], fa[i][1], fa[i][2], fa[i][3]});
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) a[i][e] = (__bf16)fa[i][e];
      }
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      if constexpr (B16) {
        b[j] = __builtin_bit_cast(bf16x8, (v4f_raw){fb[j][0], fb[j][1], fb[j][2], fb[j][3]});
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) b[j][e] = (__bf16)fb[j][e];
      }
    }
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

// Element x of an index map (strides in elements of the stored type); see
// GemmMap.  MAP = false
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
  template <int ES = 4>  // bytes per stored element
  __device__ __forceinline__ int bytes(const GemmMap& f) const { return ES * ((MAP && f.div) ? q * f.s1 + r * f.s0 : r * f.s0); }
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

// The slab of an operand stored in bf16 (autocast activations): the same
// 16-deep k slab at 2 bytes an element, moved by the same 16-byte LDS-DMA
// loads (8 elements a lane), and fragments handed to the bf16 MFMA as they
// are stored (words 0..3 of f hold the 8 values, k = 8h .. 8h + 7 as above).
//   KC slab: [BX rows][16 k] (32 bytes a row), chunk c (8 k) of row r stored
//            at chunk c ^ ((r >> 3) & 1): one 128-bit read per fragment, and
//            the 16 lanes of a read phase cover all 64 banks once;
//   XC slab: [16 k][BX] (2 BX bytes a row), the 16-byte chunk j of row k
//            stored at j ^ swz(k); a fragment is two ds_read_b64_tr_b16
//            (gfx950's transposing LDS read: lane 16g + 4a + b receives,
//            as its value e, element b of the 8 bytes that lane 16g + 4e + a
//            addresses), so lane (i, h) gets column i of k rows 8h .. 8h + 7
//            with each lane addressing one 4-element run of one k row.  swz
//            puts the four k rows a read phase touches in distinct quarters
//            of the 64 banks: rows 128 bytes (mod 256) apart alternate
//            halves by themselves (BX = 64, 192), 256-byte rows (BX = 128)
//            need all four quarters from the swizzle.
// A slab of BX = 64 is 2 KB: waves 0 and 1 issue its two loads.
template <int BX, bool KC>
struct DmaSlab16 {
  static constexpr int SIZE = BX * BK / 2;   // floats of LDS
  static constexpr int NI = BX * BK * 2 / 1024;  // 1 KB loads per slab
  static constexpr int PER_WAVE = (NI + 3) / 4;
  static constexpr int READS = KC ? 1 : 2;
  static_assert(BX % 64 == 0 && NI >= 1, "slab rows in whole 64-element runs");
  int off[PER_WAVE];

  __device__ __forceinline__ static int swz(int k) {
    return (BX / 64) % 2 ? 4 * ((k >> 1) & 1) : 4 * (k & 3);
  }
  template <bool MAP>
  __device__ __forceinline__ void init(int x0, const GemmMap& fx, const GemmMap& fk, int wave, int lane) {
#pragma unroll
    for (int q = 0; q < PER_WAVE; ++q) {
      const int c = q * 4 + wave;  // 1 KB run of the slab (c >= NI: not issued)
      if (KC) {
        const int r = c * 32 + lane / 2;
        const int chunk = (lane & 1) ^ ((r >> 3) & 1);
        off[q] = (map_at<MAP>(fx, x0 + r) + 8 * chunk) * 2;
      } else {
        const int f = c * 512 + 8 * lane;  // element of the stored slab [16][BX]
        const int k = f / BX, xs = f % BX;
        const int x = (((xs >> 3) ^ swz(k)) << 3);
        off[q] = (map_at<MAP>(fx, x0 + x) + k * fk.s0) * 2;
      }
    }
  }
#if defined(__HIP_DEVICE_COMPILE__)
  // dk: byte offset of k row/column k0 (fk(k0) * 2), uniform over the block
  __device__ __forceinline__ void issue(__amdgpu_buffer_rsrc_t rs, float* S, int wave, int dk) const {
#pragma unroll
    for (int q = 0; q < PER_WAVE; ++q)
      if (q * 4 + wave < NI)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(S + (q * 4 + wave) * 256), 16, off[q] + dk, 0, 0, 0);
  }
#endif
  __device__ __forceinline__ static void frag(const float* __restrict__ S, int xw, float f[8]) {
#if defined(__HIP_DEVICE_COMPILE__)
    const int lane = threadIdx.x & 63;
    const unsigned base = (unsigned)(uintptr_t)(const lds_float*)S;
    if (KC) {
      const int i = lane & 31, h = lane >> 5, r = xw + i;
      v4f a;
      asm volatile("ds_read_b128 %0, %1" : "=v"(a) : "v"(base + (unsigned)(r * 32 + 16 * (h ^ ((r >> 3) & 1)))));
      f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    } else {
      const int g = lane >> 4, e = (lane >> 2) & 3, a = lane & 3;
      const int x = xw + 16 * (g & 1) + 4 * a;
      const int k0 = 8 * (g >> 1) + e, k1 = k0 + 4;
      const unsigned o0 = (unsigned)(k0 * BX * 2 + ((((x >> 3) ^ swz(k0))) << 4) + (x & 7) * 2);
      const unsigned o1 = (unsigned)(k1 * BX * 2 + ((((x >> 3) ^ swz(k1))) << 4) + (x & 7) * 2);
      v2f p0, p1;
      asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(p0) : "v"(base + o0));
      asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(p1) : "v"(base + o1));
      f[0] = p0.x; f[1] = p0.y; f[2] = p1.x; f[3] = p1.y;
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
// IO (bf16 storage, bf16 MFMA only): kIoA16 / kIoB16 read A / B stored in
// bf16, kIoC16 / kIoE16 write C / E in bf16 (rounded to nearest even, the
// rounding the MFMA applies to an f32 operand) or, for EPI 2, read E in
// bf16; every layout offset counts elements of the stored type.  D and
// split-K partials stay f32.
// Split-product weight gradients on 128x128 tiles are held to 128 VGPRs (four
// workgroups per CU instead of three: the grouped q/k/v weight gradients'
// GEMM class 0.6 % faster on the C5 step, with a 20-byte spill).
template <int TM, int TN, bool TA, bool TB, bool MAP, int EPI = 0, bool BF = false, int IO = 0, bool X3 = false>
__global__ __launch_bounds__(256, (X3 && TA && TM * TN == 4) ? 4 : 2) void k_sgemm_dma(const float* __restrict__ A, const float* __restrict__ B,
                                                      float* __restrict__ C, int M, int N, int K, GemmLayouts L,
                                                      int k_chunk, int tiles_n, long split_stride,
                                                      const float* __restrict__ D, float* __restrict__ E) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int BM = 64 * TM, BN = 64 * TN;
  constexpr bool A16 = IO & kIoA16, B16 = IO & kIoB16, C16 = IO & kIoC16, E16 = IO & kIoE16, B3 = IO & kIoB3;
  static_assert(BF || IO == 0, "bf16 storage runs on the bf16 MFMA");
  static_assert(!B3 || (X3 && !B16 && !A16), "a split copy of B feeds the split product");
  constexpr int ESA = A16 ? 2 : 4, ESB = (B16 || B3) ? 2 : 4;
  constexpr int NPB = B3 ? 3 : 1;  // planes of B (its h, m and l pieces)
  // A [M][K] and B^T [N][K] are k-contiguous
  using SlabA = std::conditional_t<A16, DmaSlab16<BM, !TA>, DmaSlab<BM, !TA>>;
  using SlabB = std::conditional_t<B16 || B3, DmaSlab16<BN, TB>, DmaSlab<BN, TB>>;
  // Two-stage ring of KS 16-deep slabs per stage: stage st + 1 is in
  // flight while stage st is consumed.  Under autocast (BF) a slab's MFMA
  // work is one bf16 instruction per accumulator, so the barrier and the
  // fragment reads dominate; two slabs per stage halve the barriers and let
  // the second slab's reads overlap the first slab's MFMAs (f32 K steps are
  // long enough that one slab per stage measured faster).
  // (Three- and four-stage rings measured no faster for either precision.)
  constexpr bool BFS = BF && !X3 && (BM + BN <= 256);
  constexpr int NS = 2, KS = BFS ? 2 : 1;
  constexpr int PER_SLAB = SlabA::PER_WAVE + NPB * SlabB::PER_WAVE;  // DMA instructions per slab and wave
  // LDS reads of one slab's fragments (lgkmcnt is 4 bits)
  constexpr int READS = TM * SlabA::READS + NPB * TN * SlabB::READS;
  __shared__ __attribute__((aligned(1024))) float As[NS][KS][SlabA::SIZE];
  __shared__ __attribute__((aligned(1024))) float Bs[NS][KS][NPB * SlabB::SIZE];  // plane p at p * SIZE

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
  const long coff = map_at<MAP>(L.c.b, b);
  float* __restrict__ Cf = C + coff + (long)split * split_stride;
  __bf16* __restrict__ Ch = reinterpret_cast<__bf16*>(C) + coff;  // C16: no split
  if (D) D += coff;
  float* __restrict__ Ef = (EPI == 1 || EPI == 2) ? E + coff : E;
  __bf16* __restrict__ Eh = (EPI == 1 || EPI == 2) ? reinterpret_cast<__bf16*>(E) + coff : nullptr;
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
    const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(reinterpret_cast<const float*>(reinterpret_cast<const char*>(Ap) + (long)ba * ESA),
                                                  (unsigned)((L.ext_a - ba) * ESA));
    const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(reinterpret_cast<const float*>(reinterpret_cast<const char*>(Bp) + (long)bb * ESB),
                                                  (unsigned)(((long)NPB * L.ext_b - bb) * ESB));
    const int plane_bytes = L.ext_b * ESB;  // B3: the m and l planes follow h
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
          sa.issue(ra, As[buf][u], wave, ka.template bytes<ESA>(fak));
#pragma unroll
          for (int p = 0; p < NPB; ++p)
            sb.issue(rb, Bs[buf][u] + p * SlabB::SIZE, wave, kb.template bytes<ESB>(fbk) + p * plane_bytes);
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
      float fa[KS][TM][8], fb[KS][NPB * TN][8];
#pragma unroll
      for (int i = 0; i < TM; ++i) SlabA::frag(As[cur][0], wm + 32 * i, fa[0][i]);
#pragma unroll
      for (int p = 0; p < NPB; ++p)
#pragma unroll
        for (int j = 0; j < TN; ++j) SlabB::frag(Bs[cur][0] + p * SlabB::SIZE, wn + 32 * j, fb[0][p * TN + j]);
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
        for (int j = 0; j < NPB * TN; ++j)
          SlabB::frag(Bs[cur][KS - 1] + (j / TN) * SlabB::SIZE, wn + 32 * (j % TN), fb[KS - 1][j]);
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
      if constexpr (B3) mfma_kstep_b3<TM, TN>(fa[0], fb[0], acc);
      else mfma_kstep<TM, TN, BF, A16, B16, X3>(fa[0], fb[0], acc);
      __builtin_amdgcn_s_setprio(0);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (KS == 2) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        if (two) {
          __builtin_amdgcn_s_setprio(1);
          if constexpr (B3) mfma_kstep_b3<TM, TN>(fa[KS - 1], fb[KS - 1], acc);
          else mfma_kstep<TM, TN, BF, A16, B16, X3>(fa[KS - 1], fb[KS - 1], acc);
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
  auto pre_load = [&](int o) -> float {  // D, or for EPI 2 the GELU input E
    if constexpr (EPI == 2) return E16 ? (float)Eh[o] : Ef[o];
    else return D[o];
  };
  v16f pre[PF ? TM : 1][PF ? TN : 1];
  if (PF && (EPI == 2 || D))
    for_each([&](int i, int j, int r, bool live, int o) {
      if (PF) pre[i][j][r] = live ? pre_load(o) : 0.0f;
    });
  auto pre_at = [&](int i, int j, int r, int o) -> float {
    if constexpr (PF) return pre[i][j][r];
    else return pre_load(o);
  };
  auto store_c = [&](int o, float v) {
    if constexpr (C16) Ch[o] = (__bf16)v;
    else Cf[o] = v;
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
      if (live) store_c(o, tot[i][j][r]);
    });
  } else {
    run_k(A, B);
    for_each([&](int i, int j, int r, bool live, int o) {
      if (live) {
        float v = acc[i][j][r];
        if (EPI == 2) v = gelu_bwd(pre_at(i, j, r, o), v);
        store_c(o, D ? (EPI == 2 ? D[o] : pre_at(i, j, r, o)) + v : v);
        if constexpr (EPI == 1) {
          if constexpr (E16) Eh[o] = (__bf16)gelu_fwd(v);
          else Ef[o] = gelu_fwd(v);
        }
      }
    });
  }
#endif
}

}  // namespace
}  // namespace k
}  // namespace malus
