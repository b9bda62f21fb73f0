// The LDS-DMA GEMM instances whose B operand is a weight's split copy (the
// three bf16 planes of its h, m and l pieces, kIoB3), for split f32
// products: the forward products (neither operand transposed), which then
// split only A.  A translation unit of its own so the GEMM units build in
// parallel.
#include "k_gemm_dma.h"

namespace malus {
namespace k {
namespace {

template <int TM, int TN, bool MAP, int EPI>
const void* inst() {
  return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, false, false, MAP, EPI, true, kIoB3, true>);
}

// Variant bits as in k_gemm.hip: 8 transA, 4 transB, 32 mapped operands,
// 64 GELU epilogues, 128 grouped accumulation.
template <int TM, int TN>
const void* x3_instance(int v) {
  if (v & (8 | 4 | 128)) return nullptr;             // the forward products only
  if (v & 64) return inst<TM, TN, false, 1>();         // h = x W1, gelu(h)
  if (v & 32) return inst<TM, TN, true, 0>();          // the head projections
  return inst<TM, TN, false, 0>();                     // out = x + att Wo, x2 + ge W2
}

}  // namespace

const void* gemm_io_x3_kernel(int ti, int v) {
  switch (ti) {  // the host's tile table: 128x192, 128x128, 128x64, 64x128, 64x64
    case 0: return x3_instance<2, 3>(v);
    case 1: return x3_instance<2, 2>(v);
    case 2: return x3_instance<2, 1>(v);
    case 3: return x3_instance<1, 2>(v);
    default: return x3_instance<1, 1>(v);
  }
}

}  // namespace k
}  // namespace malus
