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
// A lane splits its 8 values of a slab with one v_cvt_pk_bf16_f32 per pair
// and piece, and a shift or mask plus a subtraction per residual (5.5 VALU
// instructions per value; a v_dot2_f32_bf16 form of the residual, 3.5 per
// value, measured 0.4 % slower on the C5 step).
//
// Non-finite operands: an infinite value's residual is inf - inf = NaN, so
// every output an infinite operand reaches is NaN (the FP32 MFMA gives
// +-inf where no inf * 0 or inf - inf arises).
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

// The bf16 value in the low / high half-word of p, as f32.
__device__ __forceinline__ float bf16_low(unsigned p) { return __builtin_bit_cast(float, p << 16); }
__device__ __forceinline__ float bf16_high(unsigned p) { return __builtin_bit_cast(float, p & 0xffff0000u); }

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
    const float ra = f[2 * q] - bf16_low(hp[q]), rb = f[2 * q + 1] - bf16_high(hp[q]);
    mp[q] = pack_bf16(ra, rb);
    lp[q] = pack_bf16(ra - bf16_low(mp[q]), rb - bf16_high(mp[q]));
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
// same sums in the same order.  x3_step issues piece product STEP (0..5)
// for every accumulator; x3_slab issues all six.
template <bool SWAP, int STEP, int TM, int TN>
__device__ __forceinline__ void x3_step(const Split3 (&a)[TM], const Split3 (&b)[TN], v16f (&acc)[TM][TN]) {
  // pieces (of the GEMM's A, of the GEMM's B) per step
  constexpr int PA = STEP == 0 ? 2 : STEP == 1 ? 0 : STEP == 2 ? 1 : STEP == 3 ? 1 : STEP == 4 ? 0 : 0;
  constexpr int PB = STEP == 0 ? 0 : STEP == 1 ? 2 : STEP == 2 ? 1 : STEP == 3 ? 0 : STEP == 4 ? 1 : 0;
  constexpr int XA = SWAP ? PB : PA, XB = SWAP ? PA : PB;  // the caller's operands
  auto piece = [](const Split3& s, int which) -> const bf16x8& { return which == 0 ? s.h : which == 1 ? s.m : s.l; };
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(piece(a[i], XA), piece(b[j], XB), acc[i][j], 0, 0, 0);
}

template <bool SWAP, int TM, int TN>
__device__ __forceinline__ void x3_slab(const Split3 (&a)[TM], const Split3 (&b)[TN], v16f (&acc)[TM][TN]) {
  x3_step<SWAP, 0>(a, b, acc);
  x3_step<SWAP, 1>(a, b, acc);
  x3_step<SWAP, 2>(a, b, acc);
  x3_step<SWAP, 3>(a, b, acc);
  x3_step<SWAP, 4>(a, b, acc);
  x3_step<SWAP, 5>(a, b, acc);
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


}  // namespace k
}  // namespace malus
