// The f32 product on the bf16 MFMA (v_mfma_f32_32x32x16_bf16), shared by
// the GEMM kernels and the fused attention kernels so that both give the
// same bits for the same 16-deep slabs.
//
// Each f32 operand value x splits exactly into three bf16 pieces,
// x = h + m + l: h = bf16(x), m = bf16(x - h), l = x - h - m, each rounded
// to nearest even.  x - h and x - h - m are f32 values (the low bits of x),
// so the residuals are exact; l has at most 8 significant bits, so it is a
// bf16 value.  The product a b is the sum of the nine piece products, each
// exact in f32 (8 x 8 significant bits).  Six are kept: hh, hm, mh, hl, lh
// and mm.  The dropped ml + lm + ll are at most 2^-23 |a b| (|m| <= 2^-8 |x|,
// |l| <= 2^-16 |x|), with random signs, near f32's unit roundoff.  Every
// piece product accumulates in f32 inside the MFMA, smallest first within a
// slab, so one 16-deep slab rounds six times where the FP32 MFMA
// (v_mfma_f32_32x32x2_f32, 8 steps of 2) rounds eight times.
//
// Non-finite operands: an infinite value's residual is inf - inf = NaN, and
// the residual of its pair partner (the other half of the same packed word)
// takes 0 * inf = NaN as well, so every output an infinite operand reaches
// is NaN (the FP32 MFMA gives +-inf where no inf * 0 or inf - inf arises).
#pragma once

#include "common.h"

namespace malus {
namespace k {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two f32 values rounded to bf16 (nearest even) in one v_cvt_pk_bf16_f32:
// a in the low half-word, b in the high one.
__device__ __forceinline__ unsigned pack_bf16(float a, float b) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(unsigned, __builtin_convertvector((f32x2){a, b}, bf16x2));
}

// x minus the bf16 value in the low (HI = false) or high half of p, in one
// v_dot2_f32_bf16 (p . (-1, 0) + x): exact whenever the difference is an
// f32 value, as the split's residuals are.  The (-1, 0) / (0, -1) operand
// sits in a register: the compiler would otherwise encode it as an inline
// constant, which this operand does not read as that bf16 pair.
template <bool HI>
__device__ __forceinline__ float minus_bf16(unsigned p, float x) {
  unsigned c;
  asm("v_mov_b32 %0, %1" : "=v"(c) : "i"(HI ? 0xbf800000u : 0x0000bf80u));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, p), __builtin_bit_cast(bf16x2, c), x, false);
}

// The three pieces of a lane's 8 fragment values, packed as the MFMA reads
// them (value e in half-word e).
struct Split3 {
  bf16x8 h, m, l;
};

__device__ __forceinline__ Split3 split3(const float (&f)[8]) {
  unsigned hp[4], mp[4], lp[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    hp[q] = pack_bf16(f[2 * q], f[2 * q + 1]);
    const float ra = minus_bf16<false>(hp[q], f[2 * q]), rb = minus_bf16<true>(hp[q], f[2 * q + 1]);
    mp[q] = pack_bf16(ra, rb);
    lp[q] = pack_bf16(minus_bf16<false>(mp[q], ra), minus_bf16<true>(mp[q], rb));
  }
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  return Split3{__builtin_bit_cast(bf16x8, (u32x4){hp[0], hp[1], hp[2], hp[3]}),
                __builtin_bit_cast(bf16x8, (u32x4){mp[0], mp[1], mp[2], mp[3]}),
                __builtin_bit_cast(bf16x8, (u32x4){lp[0], lp[1], lp[2], lp[3]})};
}

// acc[i][j] += A_i B_j over one 16-deep slab for split fragments of A (rows)
// and B (columns).  The piece products run in one order, written for the
// GEMM's A and B: (l, h), (h, l), (m, m), (m, h), (h, m), (h, h).  SWAP: the
// caller's a holds the GEMM's B and b the GEMM's A (a kernel that forms the
// transposed tile); each MFMA then takes its operands in the caller's roles
// and the same sequence of piece products, so the accumulators round the
// same sums in the same order.
template <bool SWAP, int TM, int TN>
__device__ __forceinline__ void x3_slab(const Split3 (&a)[TM], const Split3 (&b)[TN], v16f (&acc)[TM][TN]) {
#define MALUS_X3_STEP(PA, PB)                                                                          \
  _Pragma("unroll") for (int i = 0; i < TM; ++i) _Pragma("unroll") for (int j = 0; j < TN; ++j)        \
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i].PA, b[j].PB, acc[i][j], 0, 0, 0);
  if constexpr (SWAP) {
    MALUS_X3_STEP(h, l)
    MALUS_X3_STEP(l, h)
    MALUS_X3_STEP(m, m)
    MALUS_X3_STEP(h, m)
    MALUS_X3_STEP(m, h)
    MALUS_X3_STEP(h, h)
  } else {
    MALUS_X3_STEP(l, h)
    MALUS_X3_STEP(h, l)
    MALUS_X3_STEP(m, m)
    MALUS_X3_STEP(m, h)
    MALUS_X3_STEP(h, m)
    MALUS_X3_STEP(h, h)
  }
#undef MALUS_X3_STEP
}

// The same step for one accumulator (a single 32 x 32 tile).
template <bool SWAP>
__device__ __forceinline__ v16f x3_one(const Split3& a, const Split3& b, v16f c) {
  const Split3 aa[1] = {a}, bb[1] = {b};
  v16f cc[1][1] = {{c}};
  x3_slab<SWAP, 1, 1>(aa, bb, cc);
  return cc[0][0];
}

}  // namespace

// Whether f32 GEMMs (and the fused attention kernels, which reproduce the
// composed GEMMs' bits) compute their products as split bf16 pieces.
bool gemm_f32_split();

}  // namespace k
}  // namespace malus
