// The LDS-DMA GEMM instances whose B operand is a weight's bf16 copy (the
// autocast storage policy keeps one per weight matrix, refreshed each
// forward): the forward products and the dx products of the VJPs.  A
// translation unit of its own so the GEMM units build in parallel.
#include "k_gemm_dma.h"

namespace malus {
namespace k {
namespace {

template <int TM, int TN, bool TA, bool TB, bool MAP, int EPI, int IO>
const void* inst() {
  return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, TA, TB, MAP, EPI, true, IO>);
}

// Variant bits as in k_gemm.hip: 8 transA, 4 transB, 32 mapped operands,
// 64 GELU epilogues, 128 grouped accumulation; io = v >> 9 (always with
// kIoB16 here).
template <int TM, int TN>
const void* weight_instance(int v) {
  constexpr int A = kIoA16, B = kIoB16, C = kIoC16, E = kIoE16;
  const int io = (v >> 9) & 15;
  const bool ta = v & 8, tb = v & 4, mapped = v & 32, gelu = v & 64;
  if (ta) return nullptr;  // weight gradients take no weight operand
  if (v & 128) {           // the head projections' dx = dq Wq^T + dk Wk^T + dv Wv^T
    if (!tb) return nullptr;
    if (io == (A | B)) return inst<TM, TN, false, true, true, 3, A | B>();
    if (io == B) return inst<TM, TN, false, true, true, 3, B>();
    return nullptr;
  }
  if (gelu) {
    if (!tb && io == (A | B | E)) return inst<TM, TN, false, false, false, 1, A | B | E>();  // h = x W1, gelu(h)
    if (tb && io == (B | C)) return inst<TM, TN, false, true, false, 2, B | C>();          // dh = gelu_bwd(h, d W2^T)
    return nullptr;
  }
  if (mapped) {  // the head projections and, one at a time, their dx
    if (!tb && io == (A | B | C)) return inst<TM, TN, false, false, true, 0, A | B | C>();
    if (!tb && io == (A | B)) return inst<TM, TN, false, false, true, 0, A | B>();
    if (tb && io == (A | B)) return inst<TM, TN, false, true, true, 0, A | B>();
    if (tb && io == B) return inst<TM, TN, false, true, true, 0, B>();
    return nullptr;
  }
  if (!tb && io == B) return inst<TM, TN, false, false, false, 0, B>();          // out = x + att Wo
  if (!tb && io == (A | B)) return inst<TM, TN, false, false, false, 0, A | B>();  // out = x2 + ge W2
  if (tb && io == (A | B)) return inst<TM, TN, false, true, false, 0, A | B>();    // dx = dh W1^T
  if (tb && io == B) return inst<TM, TN, false, true, false, 0, B>();              // datt = d Wo^T
  return nullptr;
}

}  // namespace

const void* gemm_io_weight_kernel(int ti, int v) {
  switch (ti) {  // the host's tile table: 128x192, 128x128, 128x64, 64x128, 64x64
    case 0: return weight_instance<2, 3>(v);
    case 1: return weight_instance<2, 2>(v);
    case 2: return weight_instance<2, 1>(v);
    case 3: return weight_instance<1, 2>(v);
    default: return weight_instance<1, 1>(v);
  }
}

}  // namespace k
}  // namespace malus
