// Internal glue between the C ABI entry points: error mode, tape hooks and
// the stdlib host functions other translation units call directly.
#pragma once

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

namespace malus {

// Raised by fail() when the library runs in "return" error mode (tests);
// in the default abort mode fail() prints "malus: ..." and aborts, which is
// the reference's panic-only model (docs/adr/0006-panic-only-error-model.md).
struct MalusError : std::runtime_error {
  explicit MalusError(const char* m) : std::runtime_error(m) {}
};
void set_last_error(const char* msg);

// tape.cpp
void tape_on_release(int64_t handle);
void register_default_backward_fns();
std::vector<size_t> tape_normalize_perm(const std::vector<size_t>& raw, size_t rank);
// Record a fused node (tags 100 HeadProj, 101 Scores, 102 AttnOut,
// 103 Attention, 104 LayerNormScale, 105 GeluMatmul; see tape.cpp) with its saved handles
// and output; retains them all.
void tape_record_fused(int32_t op, const std::vector<int64_t>& saved, int64_t out, const std::vector<int64_t>& meta);

}  // namespace malus

namespace malus { struct TensorBuffer; }
// Matmul and its VJPs with an optional addend of the output's shape: returns
// D + product from one GEMM (the product rounded before the add, as a
// separate broadcast add would round it).  D == nullptr is the plain op.
int64_t matmul_impl(int64_t a, int64_t b, const malus::TensorBuffer* D);
int64_t matmul_bwd_a_impl(int64_t a, int64_t b, int64_t dout, const malus::TensorBuffer* D);
int64_t matmul_bwd_b_impl(int64_t a, int64_t b, int64_t dout, const malus::TensorBuffer* D);
int64_t layernorm_bwd_impl(int64_t y, int64_t var, int64_t dout, int64_t axis, const malus::TensorBuffer* D);
// out = layernorm(x, axis=-1) * w in one kernel, and the VJP for x (the
// layernorm VJP of dout * w, + D); the VJP for w is malus_std_mul_bwd_b(dout, y, w).
// out_bf16: out stored in bf16 (its readers being bf16 GEMMs only).
int64_t ln_affine_fwd(int64_t x, int64_t w, int64_t* y_out, int64_t* var_out, bool out_bf16 = false);
int64_t ln_affine_bwd_x(int64_t y, int64_t var, int64_t w, int64_t dout, const malus::TensorBuffer* D);
// The MLP's GELU in GEMM epilogues: h = x @ W1 with gelu(h) (returns h, 0
// when the fused GEMM does not fit), and dh = gelu_bwd(h, dout @ W2^T) (+ D).
// ge_bf16 / out_bf16: gelu(h) / dh stored in bf16 (their readers being bf16
// GEMMs only); x may be bf16.
int64_t matmul_gelu_fwd(int64_t x, int64_t w, int64_t* ge_out, bool ge_bf16 = false);
int64_t gelu_matmul_bwd_h(int64_t dout, int64_t w, int64_t h, const malus::TensorBuffer* D, bool out_bf16 = false);
// Head-folded attention GEMMs (stdlib.cpp): the composed ops' values with
// the permute copies folded into GEMM addressing.  heads_foldable: shapes
// the folded layouts support.
bool heads_foldable(size_t B, size_t T, size_t H, size_t hs);
int64_t head_proj_fwd(int64_t x, int64_t w, size_t B, size_t T, size_t H);
int64_t head_proj_bwd_x(int64_t dqh, int64_t w, size_t B, size_t T, size_t H, const malus::TensorBuffer* D);
int64_t head_proj_bwd_w(int64_t x, int64_t dqh, size_t B, size_t T, size_t H, const malus::TensorBuffer* D);
// causal: P (and dS) are lower-triangular with exact zeros above the
// diagonal, so the GEMMs skip those k slabs (same values).
// out_bf16: q, k, v stored in bf16 (for readers that round them to bf16).
void head_proj_fwd3(int64_t x, const int64_t* w, size_t B, size_t T, size_t H, int64_t* out, bool out_bf16 = false);
// Three head projections of one input together (group order = the tape's
// VJP order): the accumulated dx, and the three dW into out[0..2].
int64_t head_proj_bwd_x3(const int64_t* dqh, const int64_t* w, size_t B, size_t T, size_t H,
                         const malus::TensorBuffer* D);
void head_proj_bwd_w3(int64_t x, const int64_t* dqh, size_t B, size_t T, size_t H, int64_t* out);
int64_t attn_out_fwd(int64_t p, int64_t v, size_t B, size_t T, size_t H, bool causal);
int64_t attn_out_bwd_p(int64_t datt, int64_t v, size_t B, size_t T, size_t H, const malus::TensorBuffer* D);
int64_t attn_out_bwd_v(int64_t p, int64_t datt, size_t B, size_t T, size_t H, const malus::TensorBuffer* D,
                       bool causal);
int64_t attn_scores_bwd_impl(int64_t datt, int64_t v, int64_t p, int64_t scale, size_t B, size_t T, size_t H);
// The VJPs of two embeddings read through one gradient (the token and
// position tables of an embedding sum): *dwa, *dwb from one list launch and
// one sum launch, the same values as two malus_std_embedding_bwd calls.
// False (nothing launched) when the two do not share t, the row width and
// the i32 indices, or the shapes have no such form.
bool embedding_bwd2_impl(int64_t wa, int64_t ia, int64_t wb, int64_t ib, int64_t dout, int64_t* dwa, int64_t* dwb);
// defer_dw: dw's column combine waits for the thread's next
// k::col_combine_flush (dw unread until then).
int64_t ln_affine_bwd_xw(int64_t y, int64_t var, int64_t w, int64_t dout, const malus::TensorBuffer* D,
                         int64_t* dw_out, bool defer_dw = false);
int64_t attn_fwd_impl(int64_t q, int64_t k, int64_t v, int64_t scale, size_t B, size_t T, size_t H, int64_t* p_out);
int64_t attn_bwd_impl(int64_t datt, int64_t v, int64_t p, int64_t scale, int64_t k, const malus::TensorBuffer* D, int64_t* dq,
                      size_t B, size_t T, size_t H);
void attn_bwd_all_impl(int64_t datt, int64_t q, int64_t k, int64_t v, int64_t p, int64_t scale,
                       const malus::TensorBuffer* Dq, const malus::TensorBuffer* Dk, const malus::TensorBuffer* Dv,
                       int64_t* dq, int64_t* dk, int64_t* dv, size_t B, size_t T, size_t H);
int64_t flash_fwd_impl(int64_t q, int64_t k, int64_t v, int64_t scale, size_t B, size_t T, size_t H, int64_t* lse_out);
void flash_bwd_impl(int64_t datt, int64_t q, int64_t k, int64_t v, int64_t o, int64_t lse, int64_t scale,
                    const malus::TensorBuffer* Dq, const malus::TensorBuffer* Dk, const malus::TensorBuffer* Dv,
                    int64_t* dq, int64_t* dk, int64_t* dv, size_t B, size_t T, size_t H);
int64_t scores_bwd_q(int64_t ds, int64_t k, const malus::TensorBuffer* D, bool causal);
int64_t scores_bwd_k(int64_t ds, int64_t q, const malus::TensorBuffer* D, bool causal);

// C-ABI entry points wrap their bodies in API_TRY ... API_CATCH(value).  In
// return-error mode the outermost entry point on the thread's stack turns a
// malus error into `value` and malus_last_error(); an entry point that
// another one called passes the error on, so the caller stops where the
// error arose instead of going on with a null handle.
namespace malus {
extern thread_local int g_api_depth;
struct ApiDepth {
  ApiDepth() { ++g_api_depth; }
  ~ApiDepth() { --g_api_depth; }
};
}  // namespace malus
#define API_TRY                        \
  {                                    \
    ::malus::ApiDepth api_depth_guard_; \
    try {
#define API_CATCH(...)                                 \
  }                                                    \
  catch (const ::malus::MalusError& e) {               \
    if (::malus::g_api_depth > 1) throw;               \
    ::malus::set_last_error(e.what());                 \
    return __VA_ARGS__;                                \
  }                                                    \
  }

// Stdlib host functions (stdlib.cpp), exported with a malus_std_ prefix.
extern "C" {
int64_t malus_std_broadcast_fwd(int32_t op, int64_t a, int64_t b);
int64_t malus_std_broadcast_add_fwd(int64_t a, int64_t b);
int64_t malus_std_broadcast_sub_fwd(int64_t a, int64_t b);
int64_t malus_std_broadcast_mul_fwd(int64_t a, int64_t b);
int64_t malus_std_broadcast_div_fwd(int64_t a, int64_t b);
int64_t malus_std_scalar_op(int32_t op, int64_t a, float s, int32_t scalar_on_right);
int64_t malus_std_scalar_op_dev(int32_t op, int64_t a, int64_t s1, int32_t scalar_on_right);
int64_t malus_std_unary(int32_t op, int64_t x);
int64_t malus_std_reduce_fwd(int32_t op, int64_t x, int64_t axis, int64_t keepdim);
int64_t malus_std_reduce_all_sum_fwd(int64_t x);
int64_t malus_std_softmax_fwd(int64_t x, int64_t axis);
int64_t malus_std_layernorm_fwd(int64_t x, int64_t axis, int64_t* var_out);
int64_t malus_std_gelu_fwd(int64_t x);
int64_t malus_std_cross_entropy_fwd(int64_t logits, int64_t targets, int64_t* probs_out);
int64_t malus_std_embedding_fwd(int64_t weight, int64_t indices);
int64_t malus_std_transpose_2d_fwd(int64_t x);
int64_t malus_std_permute_3d_fwd(int64_t x, int64_t p0, int64_t p1, int64_t p2);
int64_t malus_std_permute_nd_fwd(int64_t x, int64_t p0, int64_t p1, int64_t p2, int64_t p3, int64_t p4, int64_t p5,
                                 int64_t p6, int64_t p7);
int64_t malus_std_scale_fwd(int64_t x, float c);
int64_t malus_std_fill_like_fwd(int64_t x, float c);
int64_t malus_std_eq_fwd(int64_t a, int64_t b);
int64_t malus_std_expand_axis_fwd(int64_t small, int64_t x_template, int64_t axis);
int64_t malus_std_sum_to_shape_bwd(int64_t dout, int64_t target);
int64_t malus_std_add_bwd_a(int64_t dout, int64_t a);
int64_t malus_std_add_bwd_b(int64_t dout, int64_t b);
int64_t malus_std_sub_bwd_a(int64_t dout, int64_t a);
int64_t malus_std_sub_bwd_b(int64_t dout, int64_t b);
int64_t malus_std_mul_bwd_a(int64_t dout, int64_t a, int64_t b);
int64_t malus_std_mul_bwd_b(int64_t dout, int64_t a, int64_t b);
int64_t malus_std_div_bwd_a(int64_t dout, int64_t a, int64_t b);
int64_t malus_std_div_bwd_b(int64_t dout, int64_t a, int64_t b);
int64_t malus_std_sigmoid_bwd(int64_t s, int64_t dout);
int64_t malus_std_relu_bwd(int64_t x, int64_t dout);
int64_t malus_std_tanh_bwd(int64_t t, int64_t dout);
int64_t malus_std_sqrt_bwd(int64_t s, int64_t dout);
int64_t malus_std_abs_bwd(int64_t x, int64_t dout);
int64_t malus_std_sum_bwd(int64_t x, int64_t dout);
int64_t malus_std_reduce_sum_axis_bwd(int64_t x, int64_t dout, int64_t axis);
int64_t malus_std_reduce_mean_axis_bwd(int64_t x, int64_t dout, int64_t axis);
int64_t malus_std_reduce_max_axis_bwd(int64_t x, int64_t y, int64_t dout, int64_t axis);
int64_t malus_std_reduce_var_axis_bwd(int64_t x, int64_t dout, int64_t axis);
int64_t malus_std_softmax_bwd(int64_t s, int64_t dout, int64_t axis);
int64_t malus_std_layernorm_bwd(int64_t y, int64_t var, int64_t dout, int64_t axis);
int64_t malus_std_gelu_bwd(int64_t x, int64_t dout);
int64_t malus_std_cross_entropy_bwd(int64_t probs, int64_t targets, int64_t dout);
int64_t malus_std_embedding_bwd(int64_t weight, int64_t indices, int64_t dout);
int64_t malus_std_matmul_bwd_a(int64_t a, int64_t b, int64_t dout);
int64_t malus_std_matmul_bwd_b(int64_t a, int64_t b, int64_t dout);
int64_t malus_std_adam_l2(int64_t p, int64_t g, int64_t m, int64_t v, float lr, float b1, float b2, float eps, float wd,
                          int64_t t, int64_t* m_out, int64_t* v_out);

int64_t tensor_matmul(int64_t a, int64_t b);
int64_t tensor_permute(int64_t h, const size_t* perm, size_t ndims);
int64_t tensor_reshape(int64_t h, const size_t* dims, size_t ndim);
void tape_register_backward_fn(int32_t slot, size_t fnptr);
size_t malus_tape_backward_fn(int32_t slot);
}
