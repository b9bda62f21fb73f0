/*
 * malus CPU oracle — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference runtime's host-f32 semantics
 * (crates/malus-runtime/src/metal.rs cpu_fallback loops and
 * crates/malus-runtime/src/tape.rs cpu_fallback VJPs) plus the example
 * programs' optimizer and model structure.  It is the checker for the HIP
 * product and the timed CPU baseline; nothing in the product links it.
 *
 * Every function cites the reference file:line it follows.  Tensors are
 * contiguous row-major f32 arrays; shapes are size_t arrays (rank <= 8).
 */
#ifndef MALUS_ORACLE_H
#define MALUS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- RNG (metal.rs:1690-1759) -------------------------------------------- */
void or_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
/* randn for call index `call_idx` (metal.rs:1720-1740): n standard normals. */
void or_randn(uint64_t call_idx, size_t n, float* out);
float or_rand_uniform(uint64_t call_idx);          /* metal.rs:1744-1750 */
int64_t or_rand_int(uint64_t call_idx, int64_t n); /* metal.rs:1752-1759 */
/* n successive rand_int(vocab) draws starting at call index `call_idx`. */
void or_rand_tokens(uint64_t call_idx, size_t n, int64_t vocab, int32_t* out);

/* ---- elementwise (codegen-gpu/lib.rs:373-418, metal.rs:1043-1115) ------- */
enum { OR_ADD = 0, OR_SUB = 1, OR_MUL = 2, OR_DIV = 3 };
/* __broadcast_<op>_kernel semantics with the __broadcast_<op>_fwd operand
 * swap (broadcast_binop.ml:10-112).  Output shape = the higher-rank operand's
 * shape; written to out_shape/out_ndim. */
void or_broadcast_fwd(int op, const float* a, const size_t* ash, int and_,
                      const float* b, const size_t* bsh, int bnd,
                      float* out, size_t* out_shape, int* out_ndim);
/* malus_<op>_scalar (scalar_on_right=1: a op s) / malus_r<op>_scalar (s op a). */
void or_scalar_op(int op, int scalar_on_right, const float* a, size_t n, float s, float* out);
enum { OR_RELU = 0, OR_SIGMOID, OR_TANH, OR_EXP, OR_LOG, OR_SQRT, OR_ABS, OR_GELU };
void or_unary(int op, const float* a, size_t n, float* out);

/* ---- reductions (metal.rs:1124-1271, reduce_*.ml) ----------------------- */
enum { OR_RSUM = 0, OR_RMEAN = 1, OR_RMAX = 2, OR_RVAR = 3 };
/* Output element count = outer*inner; layout identical for keepdim 0/1. */
void or_reduce_axis(int op, const float* x, const size_t* shape, int ndim, int axis, float* out);
float or_sum_all(const float* x, size_t n); /* tensor_sum metal.rs:996-1006 */
/* VJPs of the axis reductions (tape.rs:1085-1145, reduce_bwd.ml:40-71); y used by max only. */
void or_reduce_axis_bwd(int op, const float* x, const float* y, const float* dout, const size_t* shape, int ndim,
                        int axis, float* out);

/* ---- transformer ops (metal.rs:1437-1688) ------------------------------- */
void or_softmax_axis(const float* x, const size_t* shape, int ndim, int axis, float* out);
void or_layernorm_axis(const float* x, const size_t* shape, int ndim, int axis, float* out, float* var_out);
float or_cross_entropy(const float* logits, size_t n, size_t c, const int32_t* targets, float* probs_out);
void or_embedding(const float* w, size_t vocab, size_t dim, const int32_t* idx, size_t t, float* out);
void or_causal_mask(size_t t, float* out);
void or_permute(const float* x, const size_t* shape, int ndim, const size_t* perm, float* out);
void or_matmul(const float* a, const size_t* ash, int and_, const float* b, const size_t* bsh, int bnd, float* out);

/* ---- VJPs (tape.rs:971-1260) -------------------------------------------- */
void or_sum_to_shape(const float* g, const size_t* gsh, int gnd, const size_t* tsh, int tnd, float* out);
void or_unary_bwd(int op, const float* x_or_y, const float* dout, size_t n, float* out);
void or_softmax_bwd(const float* s, const float* dout, const size_t* shape, int ndim, int axis, float* out);
void or_layernorm_bwd(const float* y, const float* var, const float* dout, const size_t* shape, int ndim, int axis, float* out);
void or_cross_entropy_bwd(const float* probs, size_t n, size_t c, const int32_t* targets, float dout0, float* out);
void or_embedding_bwd(const float* dout, const int32_t* idx, size_t t, size_t dim, size_t vocab, float* out);

/* ---- optimizer (examples/nanogpt_modular.ml:97-108) ---------------------- */
void or_adam_l2_update(float* p, const float* g, float* m, float* v, size_t n,
                       float lr, float b1, float b2, float eps, float wd, int64_t t);

/* ---- workloads ----------------------------------------------------------- */
/* examples/xor.ml: returns final loss; loss_at[6] = losses at steps 0,500,1000,2000,5000,9999. */
float or_xor_train(int steps, float lr, float* loss_at, float* preds_out, float* params_out);

typedef struct or_gpt or_gpt;
/* Model of examples/nanogpt_modular.ml with L blocks and H heads. */
or_gpt* or_gpt_create(int V, int T, int C, int H, int L, int B, uint64_t rng_call_idx,
                      float lr, float b1, float b2, float eps, float wd);
void or_gpt_free(or_gpt* g);
int or_gpt_nparams(const or_gpt* g);
size_t or_gpt_param_len(const or_gpt* g, int i);
void or_gpt_get_param(const or_gpt* g, int i, float* out);
void or_gpt_get_grad(const or_gpt* g, int i, float* out);
void or_gpt_set_param(or_gpt* g, int i, const float* in);
/* AdamW moments of parameter i (which = 0: m, 1: v), to save and resume a run. */
void or_gpt_get_moment(const or_gpt* g, int i, int which, float* out);
void or_gpt_set_moment(or_gpt* g, int i, int which, const float* in);
/* forward + cross-entropy + backward; grads kept for or_gpt_get_grad. */
float or_gpt_loss_and_grads(or_gpt* g, const int32_t* x, const int32_t* y, float* logits_out);
/* full training step (forward, backward, Adam+L2 update with bias-correction step t). */
float or_gpt_step(or_gpt* g, const int32_t* x, const int32_t* y, int64_t t);
/* Worker-thread count used by the GEMM loops (OpenMP); 1 = scalar. */
void or_set_threads(int n);
int or_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
