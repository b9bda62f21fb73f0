// The LDS-DMA GEMM instances that read or write bf16-stored tensors (the
// autocast activations: layernorm outputs, the GELU output and its
// gradient), in their own translation unit so the two GEMM units build in
// parallel.  Each instance is the kernel of k_gemm_dma.h with one IO mask.
#include "k_gemm_dma.h"

namespace malus {
namespace k {
namespace {

// Variant bits as in k_gemm.hip: 8 transA, 4 transB, 32 mapped operands,
// 64 GELU epilogues, 128 grouped accumulation; io = v >> 9.
template <int TM, int TN>
const void* io_instance(int v) {
  const int io = (v >> 9) & 15;
  const bool ta = v & 8, tb = v & 4, mapped = v & 32, gelu = v & 64;
  if (v & 128) {  // the head projections' dx = dq Wq^T + dk Wk^T + dv Wv^T from bf16 dq, dk, dv
    if (!ta && tb && io == kIoA16)
      return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, false, true, true, 3, true, kIoA16>);
    return nullptr;
  }
  if (gelu) {
    // h = x W1 with ge = gelu(h) in bf16 (x the bf16 layernorm output)
    if (!ta && !tb && io == (kIoA16 | kIoE16))
      return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, false, false, false, 1, true, kIoA16 | kIoE16>);
    // dh = gelu_bwd(h, dout W2^T) in bf16
    if (!ta && tb && io == kIoC16)
      return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, false, true, false, 2, true, kIoC16>);
    return nullptr;
  }
  if (mapped) {
    // the head projections of a bf16 layernorm output (q, k, v in f32 or
    // bf16), their weight gradients (from f32 or bf16 dq) and, one
    // projection at a time, their dx
    if (!ta && !tb && io == kIoA16)
      return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, false, false, true, 0, true, kIoA16>);
    if (!ta && !tb && io == (kIoA16 | kIoC16))
      return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, false, false, true, 0, true, kIoA16 | kIoC16>);
    if (ta && !tb && io == kIoA16)
      return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, true, false, true, 0, true, kIoA16>);
    if (ta && !tb && io == (kIoA16 | kIoB16))
      return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, true, false, true, 0, true, kIoA16 | kIoB16>);
    if (!ta && tb && io == kIoA16)
      return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, false, true, true, 0, true, kIoA16>);
    return nullptr;
  }
  if (!ta && !tb && io == kIoA16)  // out = x2 + ge W2
    return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, false, false, false, 0, true, kIoA16>);
  if (!ta && tb && io == kIoA16)  // dx = dh W1^T
    return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, false, true, false, 0, true, kIoA16>);
  if (ta && !tb && io == kIoA16)  // dW2 = ge^T dout
    return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, true, false, false, 0, true, kIoA16>);
  if (ta && !tb && io == (kIoA16 | kIoB16))  // dW1 = x^T dh
    return reinterpret_cast<const void*>(&k_sgemm_dma<TM, TN, true, false, false, 0, true, kIoA16 | kIoB16>);
  return nullptr;
}

}  // namespace

const void* gemm_io_kernel(int ti, int v) {
  if ((v >> 9) & kIoB3) return gemm_io_x3_kernel(ti, v);  // a weight's split copy
  // B in bf16 outside the weight-gradient forms: a weight's bf16 copy
  if (((v >> 9) & kIoB16) && !(v & 8)) return gemm_io_weight_kernel(ti, v);
  switch (ti) {  // the host's tile table: 128x192, 128x128, 128x64, 64x128, 64x64
    case 0: return io_instance<2, 3>(v);
    case 1: return io_instance<2, 2>(v);
    case 2: return io_instance<2, 1>(v);
    case 3: return io_instance<1, 2>(v);
    default: return io_instance<1, 1>(v);
  }
}

}  // namespace k
}  // namespace malus
