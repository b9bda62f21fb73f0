// Workload drivers: the runtime-call sequences the Cranelift JIT issues for
// examples/xor.ml and examples/nanogpt_modular.ml, replayed in C++ through
// the same C ABI (tensor_matmul, the stdlib host fns, tape_record_*,
// backward, tape_get_grad ...).  Op order, tape records and operand order
// follow codegen-cpu's lowering (lib.rs:1525-1850, 2765-3082); the
// nanoGPT driver is generalized to L blocks and H heads for the C4/C5
// configurations.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <memory>
#include <vector>

#include "api.h"
#include "common.h"

extern "C" {
int64_t tensor_alloc_gpu(int32_t dtype, const size_t* shape, size_t ndim, const void* data);
int64_t tensor_alloc_ones_gpu(const size_t* shape, size_t ndim);
int64_t tensor_randn(const size_t* shape, size_t ndim);
int64_t tensor_causal_mask(int64_t t);
void tensor_release(int64_t h);
void tensor_retain(int64_t h);
float malus_tensor_get_f32(int64_t h, int64_t i);
void malus_tensor_read(int64_t h, void* dst, size_t bytes);
void tape_record_binop(int32_t op, int64_t a, int64_t b, int64_t out);
void tape_record_unary(int32_t op, int64_t x, int64_t out);
void tape_record_reduce(int32_t op, int64_t x, int64_t out, int64_t axis, int64_t keepdim);
void tape_record_perm(int32_t op, int64_t x, int64_t out, const size_t* dims, size_t ndims);
void tape_record_layernorm(int32_t op, int64_t x, int64_t out, int64_t var_h, int64_t axis);
void tape_record_cross_entropy(int32_t op, int64_t logits, int64_t out, int64_t softmax_h, int64_t targets);
void tape_record_embedding(int32_t op, int64_t weight, int64_t indices, int64_t out);
void tape_register_leaf(int64_t h);
void tape_zero_grad(const int64_t* handles, size_t count);
int64_t tape_get_grad(int64_t h);
void backward(int64_t loss);
void tape_clear(void);
void tape_pause(void);
void tape_resume(void);
int64_t kernel_dispatch(uint64_t id, const int64_t* handles, size_t count);
}

using namespace malus;

namespace {

enum Op : int32_t {
  OP_MATMUL = 0, OP_ADD = 1, OP_SUB = 2, OP_MUL = 3, OP_DIV = 4, OP_TRANSPOSE = 13, OP_RESHAPE = 19, OP_SOFTMAX = 20,
  OP_LAYERNORM = 21, OP_GELU = 22, OP_CE = 23, OP_EMBEDDING = 24,
  TAG_HEAD_PROJ = 100, TAG_SCORES = 101, TAG_ATTN_OUT = 102, TAG_ATTENTION = 103,
  TAG_LN_SCALE = 104, TAG_GELU_MATMUL = 105, TAG_FLASH = 106  // fused nodes (tape.cpp)
};

// Attention kernel choice: AUTO takes flash attention under autocast and,
// with split f32 products, from T = 256 on; else the row-register kernel
// where its shapes are built, else flash attention, else the composed ops.
enum AttnMode : int { ATTN_AUTO = 0, ATTN_FLASH = 1, ATTN_ROWS = 2, ATTN_COMPOSED = 3 };

// grad-tracked binop: lower + tape_record_binop (codegen-cpu/lib.rs:1531-1552)
int64_t binop(int32_t op, int64_t a, int64_t b) {
  int64_t out = op == OP_MATMUL ? tensor_matmul(a, b) : malus_std_broadcast_fwd(op - 1, a, b);
  tape_record_binop(op, a, b, out);
  return out;
}

int64_t reshape(int64_t x, std::initializer_list<size_t> dims) {
  std::vector<size_t> d(dims);
  int64_t out = tensor_reshape(x, d.data(), d.size());
  tape_record_unary(OP_RESHAPE, x, out);
  return out;
}

int64_t permute(int64_t x, std::initializer_list<size_t> perm) {
  std::vector<size_t> p(perm);
  int64_t out;
  if (p.size() == 3) out = malus_std_permute_3d_fwd(x, (int64_t)p[0], (int64_t)p[1], (int64_t)p[2]);  // lib.rs:3012
  else out = tensor_permute(x, p.data(), p.size());
  tape_record_perm(OP_TRANSPOSE, x, out, p.data(), p.size());
  return out;
}

int64_t layernorm(int64_t x) {
  int64_t var;
  int64_t y = malus_std_layernorm_fwd(x, 1, &var);
  tape_record_layernorm(OP_LAYERNORM, x, y, var, 1);
  return y;
}

// layernorm(x, axis=1) * w: one kernel and one LayerNormScale tape node when
// fused (the same values; y and the variance are saved for the VJPs), else
// the reference's LAYERNORM and MUL records.  *y gets the normalized rows.
// bf16_out (fused only): the product is stored in bf16 for bf16 GEMMs.
int64_t ln_scale(bool fused, int64_t x, int64_t w, int64_t* y, bool bf16_out = false) {
  if (!fused) {
    *y = layernorm(x);
    return binop(OP_MUL, *y, w);
  }
  int64_t var;
  int64_t out = ln_affine_fwd(x, w, y, &var, bf16_out);
  tape_record_fused(TAG_LN_SCALE, {x, w, *y, var}, out, {});
  tensor_release(var);  // the tape holds it
  return out;
}

// out = x + a @ w with the add in the GEMM epilogue.  The tape gets the
// reference's two records, MATMUL(a, w -> prod) and ADD(x, prod -> out);
// prod is a shape-only handle since neither VJP reads its values.
void residual_matmul(int64_t x, int64_t a, int64_t w, int64_t* prod, int64_t* out) {
  *out = matmul_impl(a, w, T(x));
  TensorBuffer* o = T(*out);
  *prod = malus::H(alloc_virtual(F32, o->shape, o->ndim));
  tape_record_binop(OP_MATMUL, a, w, *prod);
  tape_record_binop(OP_ADD, x, *prod, *out);
}

void rel(std::initializer_list<int64_t> hs) {
  for (int64_t h : hs) tensor_release(h);
}

struct Gpt {
  int V, Tn, C, H, L, B;
  float lr, b1, b2, eps, wd;
  bool fused_opt = true;
  bool fused_fwd = true;  // forward fusions: scale+mask+softmax, residual adds in GEMM epilogues (same values, same tape)
  // Parameters and moments updated in place (the same values as the
  // reference's `ps[i] = variable(new)`; the handles stay fixed, as a
  // captured step needs).  bc_dev: the bias corrections read from device
  // memory instead of kernel arguments.
  bool inplace_opt = false;
  const float* bc_dev = nullptr;
  int attn_mode = ATTN_AUTO;
  // Under autocast, the activations whose only readers are bf16 GEMMs are
  // stored in bf16 (see block_forward), and the blocks' weight matrices get
  // bf16 copies for the GEMMs (refresh_weight_copies); w16[i] is param i's.
  // With split f32 products the weight matrices get split copies instead.
  bool bf16_act = true;
  std::vector<int64_t> w16;
  std::vector<int64_t> p, m, v;  // block l params at 8l..8l+7, then wte, wpe, ln_f, lm_head
  int64_t pos = 0;               // [B*T] i32 position ids
  int64_t attn_scale = 0;        // [1,1] 1/sqrt(hs) of the fused attention (built on first use)

  int np() const { return 8 * L + 4; }
  int64_t& top(int j) { return p[8 * L + j]; }
};

// The autocast storage policy applies (below): the fused forward with the
// head-folded GEMMs, on shapes the bf16 kernels take.
bool storage_policy(const Gpt& g) {
  const size_t C = g.C, hs = C / g.H, N = (size_t)g.B * g.Tn;
  return g.bf16_act && k::autocast_on() && g.fused_fwd && heads_foldable(g.B, g.Tn, g.H, hs) && C % 128 == 0 &&
         C <= 512 && N % 8 == 0;
}

// With split f32 products (the default f32 GEMM arithmetic), outside
// autocast: the same operand copies as split copies (below), on shapes the
// split-copy kernels take.
bool split_policy(const Gpt& g) {
  return g.bf16_act && !k::autocast_on() && k::gemm_f32_split() && g.C % 16 == 0;
}

// Operand copies of the blocks' weight matrices (q, k, v, o, W1, W2) for
// the GEMMs that read them as B, refreshed in one launch at every forward;
// a copy stands for its weight only while the weight is unchanged
// (TensorBuffer::bf16_copy).
// - Under the storage policy, bf16 copies for the forward products and the
//   dx products of the VJPs: those products round their operands to bf16
//   anyway, so every value is the same, and the GEMMs move half the weight
//   bytes.
// - With split f32 products, split copies for the forward products: the
//   three bf16 planes of each value's pieces, formed once per step by the
//   split the GEMMs would run in every workgroup, so every product is the
//   same and those GEMMs split only their A operand (C5: 9.36 -> 9.26 ms;
//   the dx products read the planes slower than they split the weight).
void refresh_weight_copies(Gpt& g) {
  const bool split = split_policy(g);
  if (!split && !storage_policy(g)) return;
  if (g.w16.size() != g.p.size()) g.w16.assign(g.p.size(), 0);
  std::vector<k::Bf16Copy> segs;
  std::vector<TensorBuffer*> ws;
  for (int l = 0; l < g.L; ++l)
    for (int j : {1, 2, 3, 4, 6, 7}) {
      const size_t i = 8 * (size_t)l + j;
      TensorBuffer* w = T(g.p[i]);
      if (w->dtype != F32) continue;
      if (g.w16[i] && T(g.w16[i])->split3 != split) {  // the other kind: replace it
        TensorBuffer* old = T(g.w16[i]);
        if (w->bf16_copy == old) {
          w->bf16_copy = nullptr;
          release(old);
        }
        rel({g.w16[i]});
        g.w16[i] = 0;
      }
      if (!g.w16[i]) {
        TensorBuffer* c;
        if (split) {  // storage for three planes; the tensor describes plane h, in the weight's layout
          const size_t n3[1] = {3 * w->len};
          c = alloc_tensor(BF16, n3, 1);
          c->ndim = w->ndim;
          for (int d = 0; d < w->ndim; ++d) c->shape[d] = w->shape[d];
          c->len = w->len;
          c->split3 = true;
        } else {
          c = alloc_tensor(BF16, w->shape, w->ndim);
        }
        g.w16[i] = malus::H(c);
      }
      TensorBuffer* c = T(g.w16[i]);
      if (w->bf16_copy != c) {  // the weight's handle is new (updates that replace it)
        retain(c);
        if (w->bf16_copy) release(w->bf16_copy);
        w->bf16_copy = c;
      }
      segs.push_back(k::Bf16Copy{w->f32(), c->data(), w->len});
      ws.push_back(w);
    }
  if (segs.empty()) return;
  if (split) k::to_split3_multi(segs.data(), (int)segs.size(), stream());
  else k::to_bf16_multi(segs.data(), (int)segs.size(), stream());
  const uint64_t seq = enqueue_mark(split ? "weights_split3" : "weights_bf16");
  for (TensorBuffer* w : ws) {
    TensorBuffer* c = w->bf16_copy;
    c->write_seq = seq;
    c->copy_of = w;
    c->copy_seq = w->write_seq;
  }
}

int64_t block_forward(Gpt& g, int l, int64_t x) {
  const size_t B = g.B, Tn = g.Tn, C = g.C, H = g.H, hs = C / H, N = B * Tn;
  int64_t* P = &g.p[8 * l];
  // Fused heads: the head fold / unfold permutes and K's transpose are
  // folded into GEMM addressing (one tape node per projection, per score
  // product and per attention output; the same values as the composed ops).
  const bool fused_heads = g.fused_fwd && heads_foldable(B, Tn, H, hs);
  // The autocast storage policy (docs/adr/0037-bf16-autocast.md:8: matmuls
  // and forward elementwise kernels in bf16): the two layernorm-scale
  // outputs, gelu(h), the GELU VJP's dh and, with flash attention, q, k, v
  // and their gradients are read only as bf16 MFMA operands, which are
  // rounded to bf16 anyway, so the kernels that produce them store bf16;
  // every value of the step is unchanged, and their readers move half the
  // bytes.  h (the GELU VJP's input), the attention output (its VJP's
  // rowsum(dO * O) is f32 arithmetic), the residual stream, parameters,
  // gradients and optimizer state stay f32.
  const bool bf_act = storage_policy(g);
  // nanogpt_modular.ml:47-68
  int64_t y1;
  int64_t xn1 = ln_scale(g.fused_fwd, x, P[0], &y1, bf_act);
  auto head_fold = [&](int64_t w) {
    if (fused_heads) {
      int64_t Qh = head_proj_fwd(xn1, w, B, Tn, H);
      tape_record_fused(TAG_HEAD_PROJ, {xn1, w}, Qh, {(int64_t)B, (int64_t)Tn, (int64_t)H});
      return Qh;
    }
    int64_t q = binop(OP_MATMUL, xn1, w);
    int64_t q4 = reshape(q, {B, Tn, H, hs});
    int64_t qp = permute(q4, {0, 2, 1, 3});
    int64_t Q = reshape(qp, {B * H, Tn, hs});
    rel({q, q4, qp});
    return Q;
  };
  const bool rows_ok = fused_heads && k::attn_scores_supported(B * H, Tn, hs);
  const bool flash_ok = fused_heads && k::flash_supported(B * H, Tn, hs);
  // AUTO: flash attention under autocast (its products on the bf16 MFMA)
  // and, with split f32 products, from T = 256 on (C5: 8.90-8.92 against
  // 8.94 ms/step with the row-register kernels, three interleaved pairs; P,
  // 9/16 of [B*H, T, T] f32 a layer, is never written); else the
  // row-register kernel where it is built (with the FP32 MFMA's products its
  // backward, which reads the stored P, is the faster one).
  const bool auto_flash = !rows_ok || k::autocast_on() || (k::gemm_f32_split() && Tn >= 256);
  const bool flash = flash_ok && (g.attn_mode == ATTN_FLASH || (g.attn_mode == ATTN_AUTO && auto_flash));
  const bool fused_attention = !flash && rows_ok && (g.attn_mode == ATTN_AUTO || g.attn_mode == ATTN_ROWS);
  // Under the storage policy flash attention reads q, k, v only as bf16 MFMA
  // operands, and their gradients feed only bf16 GEMMs: all six in bf16.
  const bool qkv_bf16 = bf_act && flash;
  int64_t Q, K, Vv;
  if (fused_heads) {  // the three projections in one grouped launch, three tape nodes
    const int64_t w[3] = {P[1], P[2], P[3]};
    int64_t qkv[3];
    head_proj_fwd3(xn1, w, B, Tn, H, qkv, qkv_bf16);
    for (int i = 0; i < 3; ++i) tape_record_fused(TAG_HEAD_PROJ, {xn1, w[i]}, qkv[i], {(int64_t)B, (int64_t)Tn, (int64_t)H});
    Q = qkv[0];
    K = qkv[1];
    Vv = qkv[2];
  } else {
    Q = head_fold(P[1]);
    K = head_fold(P[2]);
    Vv = head_fold(P[3]);
  }
  int64_t Kt = fused_heads ? 0 : permute(K, {0, 2, 1});
  int64_t scale;
  if (fused_attention || flash) {
    // variable(ones(1,1) * (1/sqrt(hs))) is the same value every forward and
    // receives no gradient in the fused form: build it once per model
    if (!g.attn_scale) {
      size_t s11[2] = {1, 1};
      int64_t ones11 = tensor_alloc_ones_gpu(s11, 2);
      g.attn_scale = malus_std_scalar_op(k::MUL, ones11, 1.0f / sqrtf((float)hs), 1);
      tensor_release(ones11);
    }
    scale = g.attn_scale;
    tensor_retain(scale);
  } else {
    size_t s11[2] = {1, 1};
    int64_t ones11 = tensor_alloc_ones_gpu(s11, 2);
    scale = malus_std_scalar_op(k::MUL, ones11, 1.0f / sqrtf((float)hs), 1);  // ones(1,1) * (1/sqrt(hs))
    tensor_release(ones11);
    tape_register_leaf(scale);  // variable(...)
  }
  const size_t sshape[3] = {B * H, Tn, Tn};
  int64_t S = 0, mask = 0, Ss = 0, Sm = 0, Pm = 0, AO = 0, ao4 = 0, aop = 0, att;
  if (flash) {
    // Flash attention: the same value with an online softmax; neither the
    // scores nor the probabilities exist, the VJP recomputes them from the
    // saved row log-sum-exp.
    int64_t lse = 0;
    att = flash_fwd_impl(Q, K, Vv, scale, B, Tn, H, &lse);
    tape_record_fused(TAG_FLASH, {Q, K, Vv, att, lse, scale}, att, {(int64_t)B, (int64_t)Tn, (int64_t)H});
    tensor_release(lse);
  } else if (fused_attention) {
    // Fused causal attention: S = Q @ K^T, scale, causal mask, softmax (P
    // stored) and att = P @ V written straight into [B*T, C], all in one
    // kernel, and one tape node whose VJP runs the fused scores backward.
    // The causal mask is computed in the kernels, so its tensor is not built;
    // the scale and mask leaves of the composed form are released before
    // backward and never receive gradients.
    att = attn_fwd_impl(Q, K, Vv, scale, B, Tn, H, &Pm);
    tape_record_fused(TAG_ATTENTION, {Q, K, Vv, Pm, scale}, att, {(int64_t)B, (int64_t)Tn, (int64_t)H});
  } else {
    if (fused_heads) {  // S = Q @ K^T with K read in place
      TensorBuffer* st = alloc_tensor(F32, sshape, 3);
      KTimer* kt = ktimer_begin("gemm");
      k::gemm(T(Q)->f32(), T(K)->f32(), st->f32(), (int)(B * H), (int)Tn, (int)Tn, (int)hs, false, true,
              (long)(Tn * hs), (long)(Tn * hs), (long)(Tn * Tn), stream());
      ktimer_end(kt, 2.0 * B * H * Tn * Tn * hs);
      st->write_seq = enqueue_mark("matmul");
      S = malus::H(st);
      tape_record_fused(TAG_SCORES, {Q, K}, S, {});
    } else {
      S = binop(OP_MATMUL, Q, Kt);
    }
    mask = tensor_causal_mask((int64_t)Tn);
    tape_register_leaf(mask);  // variable(mask)
    if (g.fused_fwd) {
      // scores * scale + mask -> softmax in one pass.  The tape gets the same
      // three records; the two intermediates are shape-only handles because
      // no VJP reads their values (add: shapes; mul: S and scale; softmax: P).
      TensorBuffer* st = T(S);
      Ss = malus::H(alloc_virtual(F32, st->shape, st->ndim));
      Sm = malus::H(alloc_virtual(F32, st->shape, st->ndim));
      TensorBuffer* p = alloc_tensor(F32, st->shape, st->ndim);
      k::scale_mask_softmax(st->f32(), T(scale)->f32(), T(mask)->f32(), p->f32(), st->len / Tn, Tn, Tn, stream());
      p->write_seq = enqueue_mark("scale_mask_softmax");
      Pm = malus::H(p);
      tape_record_binop(OP_MUL, S, scale, Ss);
      tape_record_binop(OP_ADD, Ss, mask, Sm);
    } else {
      Ss = binop(OP_MUL, S, scale);
      Sm = binop(OP_ADD, Ss, mask);
      Pm = malus_std_softmax_fwd(Sm, 2);
    }
    tape_record_reduce(OP_SOFTMAX, Sm, Pm, 2, 0);
    if (fused_heads) {
      att = attn_out_fwd(Pm, Vv, B, Tn, H, false);
      tape_record_fused(TAG_ATTN_OUT, {Pm, Vv}, att, {(int64_t)B, (int64_t)Tn, (int64_t)H});
    } else {
      AO = binop(OP_MATMUL, Pm, Vv);
      ao4 = reshape(AO, {B, H, Tn, hs});
      aop = permute(ao4, {0, 2, 1, 3});
      att = reshape(aop, {N, C});
    }
  }
  int64_t proj, x2;
  if (g.fused_fwd) residual_matmul(x, att, P[4], &proj, &x2);
  else {
    proj = binop(OP_MATMUL, att, P[4]);
    x2 = binop(OP_ADD, x, proj);
  }
  int64_t y2;
  int64_t xn2 = ln_scale(g.fused_fwd, x2, P[5], &y2, bf_act);
  int64_t ge = 0, mo, x3;
  int64_t h = g.fused_fwd ? matmul_gelu_fwd(xn2, P[6], &ge, bf_act) : 0;
  if (h) {
    // MLP: gelu in the first GEMM's epilogue; out = x2 + ge @ W2 with the add
    // in the second's.  Tape: MATMUL(xn2, W1 -> h), GeluMatmul(h, W2; ge ->
    // prod) whose VJP applies the GELU VJP in the dA GEMM's epilogue, and
    // ADD(x2, prod -> out); prod is shape-only.
    tape_record_binop(OP_MATMUL, xn2, P[6], h);
    x3 = matmul_impl(ge, P[7], T(x2));
    TensorBuffer* o = T(x3);
    mo = malus::H(alloc_virtual(F32, o->shape, o->ndim));
    tape_record_fused(TAG_GELU_MATMUL, {h, P[7], ge}, mo, {});
    tape_record_binop(OP_ADD, x2, mo, x3);
  } else {
    h = binop(OP_MATMUL, xn2, P[6]);
    ge = malus_std_gelu_fwd(h);
    tape_record_unary(OP_GELU, h, ge);
    if (g.fused_fwd) residual_matmul(x2, ge, P[7], &mo, &x3);
    else {
      mo = binop(OP_MATMUL, ge, P[7]);
      x3 = binop(OP_ADD, x2, mo);
    }
  }
  rel({y1, xn1, Q, K, Vv, Kt, scale, S, Ss, mask, Sm, Pm, AO, ao4, aop, att, proj, x2, y2, xn2, h, ge, mo});
  return x3;
}

// GPT.forward (nanogpt_modular.ml:75-91) + cross_entropy (lib.rs:2945-2972)
int64_t gpt_forward_loss(Gpt& g, int64_t toks, int64_t targets, int64_t* logits_out) {
  refresh_weight_copies(g);
  int64_t te, pe, x;
  TensorBuffer *wte = T(g.top(0)), *wpe = T(g.top(1)), *tk = T(toks), *ps = T(g.pos);
  if (g.fused_fwd && tk->dtype == I32 && ps->dtype == I32 && tk->ndim == 1 && tk->len == ps->len &&
      wte->shape[1] == wpe->shape[1] && wte->shape[1] % 4 == 0) {
    // tok_emb + pos_emb in one pass; the tape gets the same three records,
    // with the two embeddings as shape-only handles (their VJPs read the
    // indices and the gradient, the add's reads shapes)
    const size_t d = wte->shape[1], sh[2] = {tk->len, d};
    TensorBuffer* xo = alloc_tensor(F32, sh, 2);
    k::embedding2(wte->f32(), tk->i32(), wte->shape[0], wpe->f32(), ps->i32(), wpe->shape[0], xo->f32(), tk->len, d,
                  device_error_flag(), stream());
    xo->write_seq = enqueue_mark("embedding2");
    te = malus::H(alloc_virtual(F32, sh, 2));
    pe = malus::H(alloc_virtual(F32, sh, 2));
    x = malus::H(xo);
    tape_record_embedding(OP_EMBEDDING, g.top(0), toks, te);
    tape_record_embedding(OP_EMBEDDING, g.top(1), g.pos, pe);
    tape_record_binop(OP_ADD, te, pe, x);
  } else {
    te = malus_std_embedding_fwd(g.top(0), toks);
    tape_record_embedding(OP_EMBEDDING, g.top(0), toks, te);
    pe = malus_std_embedding_fwd(g.top(1), g.pos);
    tape_record_embedding(OP_EMBEDDING, g.top(1), g.pos, pe);
    x = binop(OP_ADD, te, pe);
  }
  rel({te, pe});
  for (int l = 0; l < g.L; ++l) {
    int64_t nx = block_forward(g, l, x);
    tensor_release(x);
    x = nx;
  }
  int64_t yf;
  int64_t xf = ln_scale(g.fused_fwd, x, g.top(2), &yf);
  int64_t logits = binop(OP_MATMUL, xf, g.top(3));
  rel({x, yf, xf});
  if (!targets) {
    *logits_out = logits;
    return 0;
  }
  int64_t probs;
  int64_t loss = malus_std_cross_entropy_fwd(logits, targets, &probs);
  tape_record_cross_entropy(OP_CE, logits, loss, probs, targets);
  if (logits_out) *logits_out = logits;
  else tensor_release(logits);
  return loss;
}

// adamw (nanogpt_modular.ml:97-108) for params [beg, end).  The fused form
// updates every tensor in one multi-tensor launch with the same per-element
// expression tree as the op-by-op sequence the JIT emits.
void adamw_range(Gpt& g, int beg, int end, int64_t t) {
  const float bc1 = 1.0f - powf(g.b1, (float)t), bc2 = 1.0f - powf(g.b2, (float)t);
  if (g.inplace_opt) {
    std::vector<k::AdamSeg> segs;
    std::vector<int64_t> grads;
    for (int i = beg; i < end; ++i) {
      int64_t grad = tape_get_grad(g.p[i]);
      grads.push_back(grad);
      TensorBuffer *tp = T(g.p[i]), *tg = T(grad), *tm = T(g.m[i]), *tv = T(g.v[i]);
      if (tg->len != tp->len || tm->len != tp->len || tv->len != tp->len) fail("malus: adam update: length mismatch");
      // each element is read before the same thread writes it back
      segs.push_back(k::AdamSeg{tp->f32(), tg->f32(), tm->f32(), tv->f32(), tp->f32(), tm->f32(), tv->f32(), tp->len});
    }
    k::adam_l2_multi(segs.data(), (int)segs.size(), g.lr, g.b1, g.b2, 1.0f - g.b1, 1.0f - g.b2, bc1, bc2, g.eps, g.wd,
                     stream(), g.bc_dev);
    const uint64_t seq = enqueue_mark("adam");
    for (int i = beg; i < end; ++i) {
      T(g.p[i])->write_seq = T(g.m[i])->write_seq = T(g.v[i])->write_seq = seq;
      tensor_release(grads[i - beg]);
    }
    return;
  }
  if (g.fused_opt) {
    std::vector<k::AdamSeg> segs;
    std::vector<int64_t> grads, np_(end - beg), nm(end - beg), nv(end - beg);
    for (int i = beg; i < end; ++i) {
      int64_t grad = tape_get_grad(g.p[i]);
      grads.push_back(grad);
      TensorBuffer *tp = T(g.p[i]), *tg = T(grad), *tm = T(g.m[i]), *tv = T(g.v[i]);
      if (tg->len != tp->len || tm->len != tp->len || tv->len != tp->len) fail("malus: adam update: length mismatch");
      TensorBuffer *po = alloc_like(tp), *mo = alloc_like(tp), *vo = alloc_like(tp);
      np_[i - beg] = H(po);
      nm[i - beg] = H(mo);
      nv[i - beg] = H(vo);
      segs.push_back(k::AdamSeg{tp->f32(), tg->f32(), tm->f32(), tv->f32(), po->f32(), mo->f32(), vo->f32(), tp->len});
    }
    k::adam_l2_multi(segs.data(), (int)segs.size(), g.lr, g.b1, g.b2, 1.0f - g.b1, 1.0f - g.b2, bc1, bc2, g.eps, g.wd,
                     stream());
    const uint64_t seq = enqueue_mark("adam");
    for (int i = beg; i < end; ++i) {
      T(np_[i - beg])->write_seq = T(nm[i - beg])->write_seq = T(nv[i - beg])->write_seq = seq;
      tensor_release(grads[i - beg]);
      tape_register_leaf(np_[i - beg]);  // ps[i] = variable(...)
      rel({g.p[i], g.m[i], g.v[i]});
      g.p[i] = np_[i - beg];
      g.m[i] = nm[i - beg];
      g.v[i] = nv[i - beg];
    }
    return;
  }
  for (int i = beg; i < end; ++i) {
    int64_t grad = tape_get_grad(g.p[i]);
    int64_t np_, nm, nv;
    {  // the op-by-op sequence the JIT emits
      int64_t wdp = malus_std_scalar_op(k::MUL, g.p[i], g.wd, 0);
      int64_t gg = malus_std_broadcast_fwd(k::ADD, grad, wdp);
      int64_t t1 = malus_std_scalar_op(k::MUL, g.m[i], g.b1, 0);
      int64_t t2 = malus_std_scalar_op(k::MUL, gg, 1.0f - g.b1, 0);
      nm = malus_std_broadcast_fwd(k::ADD, t1, t2);
      int64_t t3 = malus_std_scalar_op(k::MUL, g.v[i], g.b2, 0);
      int64_t t4 = malus_std_scalar_op(k::MUL, gg, 1.0f - g.b2, 0);
      int64_t t5 = malus_std_broadcast_fwd(k::MUL, t4, gg);
      nv = malus_std_broadcast_fwd(k::ADD, t3, t5);
      int64_t mh = malus_std_scalar_op(k::DIV, nm, bc1, 1);
      int64_t vh = malus_std_scalar_op(k::DIV, nv, bc2, 1);
      int64_t t6 = malus_std_scalar_op(k::MUL, mh, g.lr, 0);
      int64_t t7 = malus_std_unary(k::SQRT, vh);
      int64_t t8 = malus_std_scalar_op(k::ADD, t7, g.eps, 1);
      int64_t t9 = malus_std_broadcast_fwd(k::DIV, t6, t8);
      np_ = malus_std_broadcast_fwd(k::SUB, g.p[i], t9);
      rel({wdp, gg, t1, t2, t3, t4, t5, mh, vh, t6, t7, t8, t9});
    }
    tensor_release(grad);
    tape_register_leaf(np_);  // ps[i] = variable(...)
    rel({g.p[i], g.m[i], g.v[i]});
    g.p[i] = np_;
    g.m[i] = nm;
    g.v[i] = nv;
  }
}

int64_t zeros_like_param(int64_t p) {
  TensorBuffer* t = T(p);
  TensorBuffer* z = alloc_tensor(F32, t->shape, t->ndim);
  k::fill(z->f32(), 0.0f, z->len, stream());
  z->write_seq = enqueue_mark("zeros");
  return H(z);
}

}  // namespace

extern "C" {

// Builds the model of nanogpt_modular.ml main() (lines 138-164) with L
// blocks: randn draws in the reference order (block 0..L-1: wq wk wv wo w1
// w2; then wte, wpe, lm_head), each scaled by 0.02.
void* malus_gpt_create(int V, int Tn, int C, int H, int L, int B, float lr, float b1, float b2, float eps, float wd) {
  API_TRY
  if (H <= 0 || C % H) fail("malus: n_embd %d is not divisible by n_head %d", C, H);
  auto* g = new Gpt{V, Tn, C, H, L, B, lr, b1, b2, eps, wd};
  size_t s11[2] = {1, 1};
  int64_t ones11 = tensor_alloc_ones_gpu(s11, 2);
  int64_t init_scale = malus_std_scalar_op(k::MUL, ones11, 0.02f, 1);  // ones(1,1) * 0.02
  tensor_release(ones11);
  auto randn_scaled = [&](size_t r, size_t c) {
    size_t sh[2] = {r, c};
    int64_t rn = tensor_randn(sh, 2);
    int64_t w = malus_std_broadcast_fwd(k::MUL, rn, init_scale);
    tensor_release(rn);
    tape_register_leaf(w);
    return w;
  };
  auto ones_vec = [&](size_t c) {
    size_t sh[1] = {c};
    int64_t o = tensor_alloc_ones_gpu(sh, 1);
    tape_register_leaf(o);
    return o;
  };
  const size_t Cs = (size_t)C, C4 = 4 * (size_t)C;
  for (int l = 0; l < L; ++l) {
    g->p.push_back(ones_vec(Cs));
    for (int j = 0; j < 4; ++j) g->p.push_back(randn_scaled(Cs, Cs));
    g->p.push_back(ones_vec(Cs));
    g->p.push_back(randn_scaled(Cs, C4));
    g->p.push_back(randn_scaled(C4, Cs));
  }
  g->p.push_back(randn_scaled((size_t)V, Cs));
  g->p.push_back(randn_scaled((size_t)Tn, Cs));
  g->p.push_back(ones_vec(Cs));
  g->p.push_back(randn_scaled(Cs, (size_t)V));
  tensor_release(init_scale);
  for (int64_t p : g->p) {
    g->m.push_back(zeros_like_param(p));
    g->v.push_back(zeros_like_param(p));
  }
  // position ids [B*T] (nanogpt_modular.ml:80-84), built once on the device
  size_t sh[1] = {(size_t)B * Tn};
  TensorBuffer* pos = alloc_tensor(I32, sh, 1);
  k::iota_rows(pos->i32(), (size_t)B, (size_t)Tn, stream());
  pos->write_seq = enqueue_mark("positions");
  g->pos = malus::H(pos);
  return g;
  API_CATCH(nullptr)
}

void malus_gpt_free(void* gp) {
  API_TRY
  auto* g = static_cast<Gpt*>(gp);
  if (!g) return;
  for (size_t i = 0; i < g->p.size(); ++i) rel({g->p[i], g->m[i], g->v[i]});
  for (int64_t c : g->w16) rel({c});  // a weight handle still alive elsewhere keeps its own reference
  tensor_release(g->pos);
  tensor_release(g->attn_scale);
  delete g;
  API_CATCH()
}

int malus_gpt_nparams(void* gp) { return static_cast<Gpt*>(gp)->np(); }
int64_t malus_gpt_param(void* gp, int i) { return static_cast<Gpt*>(gp)->p[(size_t)i]; }
int64_t malus_gpt_moment(void* gp, int i, int which) {
  auto* g = static_cast<Gpt*>(gp);
  return which ? g->v[(size_t)i] : g->m[(size_t)i];
}
// 1 (default): forward fusions on — scores * scale + mask -> softmax as one
// kernel, and the residual adds folded into the producing GEMM's epilogue;
// 0: every op separately.  Values and tape records are the same either way.
void malus_gpt_set_fused_forward(void* gp, int on) { static_cast<Gpt*>(gp)->fused_fwd = on != 0; }
void malus_gpt_set_bf16_activations(void* gp, int on) { static_cast<Gpt*>(gp)->bf16_act = on != 0; }

void malus_gpt_set_fused_optimizer(void* gp, int on) { static_cast<Gpt*>(gp)->fused_opt = on != 0; }
// 0: automatic, 1: flash attention, 2: the row-register fused kernel, 3: composed ops
int malus_gpt_set_attention(void* gp, int mode) {
  API_TRY
  if (mode < ATTN_AUTO || mode > ATTN_COMPOSED) fail("malus: attention mode %d is not 0..3", mode);
  static_cast<Gpt*>(gp)->attn_mode = mode;
  return 0;
  API_CATCH(-1)
}

// Forward + cross-entropy (recorded on the tape); returns the loss [1].
int64_t malus_gpt_forward_loss(void* gp, int64_t toks, int64_t targets) {
  API_TRY
  return gpt_forward_loss(*static_cast<Gpt*>(gp), toks, targets, nullptr);
  API_CATCH(0)
}

// Forward only, no tape; returns logits [B*T, V].
int64_t malus_gpt_logits(void* gp, int64_t toks) {
  API_TRY
  tape_pause();
  int64_t logits = 0;
  gpt_forward_loss(*static_cast<Gpt*>(gp), toks, 0, &logits);
  tape_resume();
  return logits;
  API_CATCH(0)
}

void malus_gpt_zero_grad(void* gp) {
  auto* g = static_cast<Gpt*>(gp);
  // zero_grad per submodule (nanogpt_modular.ml:178-182)
  for (int l = 0; l < g->L; ++l) tape_zero_grad(&g->p[8 * l], 8);
  tape_zero_grad(&g->p[8 * g->L], 4);
}

void malus_gpt_optimizer_step(void* gp, int64_t t) {
  API_TRY
  auto* g = static_cast<Gpt*>(gp);
  // lines 186-187 (each block's params), then line 188 (the rest): every
  // update is elementwise on its own tensors, so the whole list is one range
  // (the fused form then takes two multi-tensor launches)
  adamw_range(*g, 0, 8 * g->L + 4, t);
  API_CATCH()
}

// One training step (nanogpt_modular.ml:167-189 minus the host batch build):
// zero_grad, forward, cross_entropy, backward, AdamW.  Returns the loss [1]
// (owned by the caller; nothing is read back to the host).
int64_t malus_gpt_step(void* gp, int64_t toks, int64_t targets, int64_t t) {
  API_TRY
  auto* g = static_cast<Gpt*>(gp);
  malus_gpt_zero_grad(g);
  int64_t loss = gpt_forward_loss(*g, toks, targets, nullptr);
  backward(loss);
  malus_gpt_optimizer_step(g, t);
  return loss;
  API_CATCH(0)
}

// examples/xor.ml main(): returns the final loss; loss_at[6] receives the
// printed losses (steps 0, 500, 1000, 2000, 5000, 9999), preds[4] the final
// predictions, params[33] = w1 (16), b1 (8), w2 (8), b2 (1).
// `sigmoid_backward_id` is the kernel id of the user kernel xor.ml:1-2,
// registered through malus_runtime_init.
float malus_xor_run(int steps, float lr, uint64_t sigmoid_backward_id, float* loss_at, float* preds, float* params) {
  API_TRY
  const float xd[8] = {0, 0, 0, 1, 1, 0, 1, 1}, td[4] = {0, 1, 1, 0}, od[4] = {1, 1, 1, 1};
  const float w1d[16] = {0.5f, -0.6f, 0.7f, -0.4f, 0.3f, -0.5f, 0.6f, -0.3f,
                         -0.4f, 0.5f, -0.6f, 0.7f, -0.3f, 0.4f, -0.5f, 0.6f};
  const float b1d[8] = {0.1f, -0.1f, 0.1f, -0.1f, 0.1f, -0.1f, 0.1f, -0.1f};
  const float w2d[8] = {0.6f, -0.5f, 0.4f, -0.6f, 0.5f, -0.4f, 0.6f, -0.5f};
  const float b2d[1] = {0.0f};
  size_t s42[2] = {4, 2}, s41[2] = {4, 1}, s28[2] = {2, 8}, s18[2] = {1, 8}, s81[2] = {8, 1}, s11[2] = {1, 1};
  int64_t x = tensor_alloc_gpu(F32, s42, 2, xd), target = tensor_alloc_gpu(F32, s41, 2, td);
  int64_t ones41 = tensor_alloc_gpu(F32, s41, 2, od);
  int64_t w1 = tensor_alloc_gpu(F32, s28, 2, w1d), b1 = tensor_alloc_gpu(F32, s18, 2, b1d);
  int64_t w2 = tensor_alloc_gpu(F32, s81, 2, w2d), b2 = tensor_alloc_gpu(F32, s11, 2, b2d);
  const int report[6] = {0, 500, 1000, 2000, 5000, 9999};
  float loss_v = 0.0f;
  int64_t out = 0;
  for (int step = 0; step < steps; ++step) {
    int64_t a1 = tensor_matmul(x, w1), a2 = tensor_matmul(ones41, b1);
    int64_t z1 = malus_std_broadcast_fwd(k::ADD, a1, a2);
    int64_t h = malus_std_unary(k::SIGMOID, z1);
    int64_t c1 = tensor_matmul(h, w2), c2 = tensor_matmul(ones41, b2);
    int64_t z2 = malus_std_broadcast_fwd(k::ADD, c1, c2);
    if (out) tensor_release(out);
    out = malus_std_unary(k::SIGMOID, z2);
    int64_t diff = malus_std_broadcast_fwd(k::SUB, out, target);
    int64_t sq = malus_std_broadcast_fwd(k::MUL, diff, diff);
    int64_t loss = malus_std_reduce_all_sum_fwd(sq);
    for (int r = 0; r < 6; ++r)
      if (step == report[r]) {
        float lv = malus_tensor_get_f32(loss, 0);  // println reads the loss (flush)
        if (loss_at) loss_at[r] = lv;
      }
    if (step == steps - 1) loss_v = malus_tensor_get_f32(loss, 0);
    int64_t dout = malus_std_scalar_op(k::MUL, diff, 2.0f, 0);
    int64_t hs1[2] = {dout, out};
    int64_t dz2 = kernel_dispatch(sigmoid_backward_id, hs1, 2);
    int64_t hT = malus_std_transpose_2d_fwd(h);
    int64_t dw2 = tensor_matmul(hT, dz2);
    int64_t oT = malus_std_transpose_2d_fwd(ones41);
    int64_t db2 = tensor_matmul(oT, dz2);
    int64_t w2T = malus_std_transpose_2d_fwd(w2);
    int64_t dh = tensor_matmul(dz2, w2T);
    int64_t hs2[2] = {dh, h};
    int64_t dz1 = kernel_dispatch(sigmoid_backward_id, hs2, 2);
    int64_t xT = malus_std_transpose_2d_fwd(x);
    int64_t dw1 = tensor_matmul(xT, dz1);
    int64_t oT2 = malus_std_transpose_2d_fwd(ones41);
    int64_t db1 = tensor_matmul(oT2, dz1);
    auto sgd = [&](int64_t& w, int64_t dw) {
      int64_t u = malus_std_scalar_op(k::MUL, dw, lr, 0);
      int64_t nw = malus_std_broadcast_fwd(k::SUB, w, u);
      rel({u, w});
      w = nw;
    };
    sgd(w1, dw1);
    sgd(b1, db1);
    sgd(w2, dw2);
    sgd(b2, db2);
    rel({a1, a2, z1, h, c1, c2, z2, diff, sq, loss, dout, dz2, hT, dw2, oT, db2, w2T, dh, dz1, xT, dw1, oT2, db1});
  }
  if (preds && out) malus_tensor_read(out, preds, 4 * sizeof(float));
  if (params) {
    malus_tensor_read(w1, params, 16 * sizeof(float));
    malus_tensor_read(b1, params + 16, 8 * sizeof(float));
    malus_tensor_read(w2, params + 24, 8 * sizeof(float));
    malus_tensor_read(b2, params + 32, sizeof(float));
  }
  rel({x, target, ones41, w1, b1, w2, b2});
  if (out) tensor_release(out);
  return loss_v;
  API_CATCH(0.0f)
}

// ---- the training step as a HIP graph ---------------------------------------
// One step (token upload, zero_grad, forward, cross_entropy, backward, AdamW)
// captured once and replayed: one hipGraphLaunch per step instead of ~180
// kernel launches.  Whatever changes between steps comes from pinned host
// memory through the graph's own copy nodes: the token and target ids, and
// AdamW's two bias corrections (1 - b^t, computed on the host as in the
// eager step and read by the kernel from device memory).  Parameters and
// moments are updated in place, so every address the graph uses stays fixed;
// the pool keeps the buffers the captured step allocated for the graph alone
// (pool_capture_begin/end).  Values are those of the eager step.

}  // extern "C"

namespace {

struct GptGraph {
  Gpt* g = nullptr;
  int id = 0;
  size_t n = 0;                  // tokens per step (B * T)
  // Where a step's token and target ids come from: copied from host arrays
  // (`pinned` holds [n] i32 tokens, [n] i32 targets, [2] f32 bias
  // corrections), or drawn on the device (`drawn`: `pinned` holds the two
  // u64 call indices, then the [2] f32 bias corrections, copied by one node
  // into `calls`, and a kernel node draws the ids).
  bool drawn = false;
  char* pinned = nullptr;
  int64_t toks = 0, tgts = 0;    // fixed device inputs [n] i32
  int64_t calls = 0;             // drawn: [3] i64 on the device, the call indices then the bias corrections
  TensorBuffer* bc = nullptr;    // ids copied from the host: [2] f32 on the device
  int64_t loss = 0;              // written by every replay
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  hipEvent_t done = nullptr;     // after the last launch: the pinned inputs may be rewritten once it completes
  bool launched = false;
};

std::atomic<int> g_graph_ids{0};

size_t pinned_bytes(const GptGraph& gr) {
  return (gr.drawn ? 2 * sizeof(uint64_t) : 2 * gr.n * sizeof(int32_t)) + 2 * sizeof(float);
}

// Step t's inputs into the pinned block, once the last launch has read it.
void graph_set_inputs(GptGraph& gr, const int32_t* x, const int32_t* y, uint64_t cx, uint64_t cy, int64_t t) {
  if (gr.launched) MALUS_HIP(hipEventSynchronize(gr.done));  // the previous step's copies have read the buffer
  float* bc;
  if (gr.drawn) {
    uint64_t* calls = reinterpret_cast<uint64_t*>(gr.pinned);
    calls[0] = cx;
    calls[1] = cy;
    bc = reinterpret_cast<float*>(calls + 2);
  } else {
    int32_t* ids = reinterpret_cast<int32_t*>(gr.pinned);
    memcpy(ids, x, gr.n * sizeof(int32_t));
    memcpy(ids + gr.n, y, gr.n * sizeof(int32_t));
    bc = reinterpret_cast<float*>(ids + 2 * gr.n);
  }
  bc[0] = 1.0f - powf(gr.g->b1, (float)t);  // nanogpt_modular.ml:99-100, as adamw_range computes them
  bc[1] = 1.0f - powf(gr.g->b2, (float)t);
}

// The step's work on the stream; the same calls eagerly and under capture.
int64_t graph_step_body(GptGraph& gr, int64_t t) {
  Gpt& g = *gr.g;
  if (gr.drawn) {
    MALUS_HIP(hipMemcpyAsync(T(gr.calls)->data(), gr.pinned, pinned_bytes(gr), hipMemcpyHostToDevice, stream()));
    k::rand_tokens(T(gr.toks)->i32(), T(gr.tgts)->i32(), gr.n, static_cast<const uint64_t*>(T(gr.calls)->data()), 0,
                   0, (uint32_t)g.V, stream());
  } else {
    const int32_t* ids = reinterpret_cast<const int32_t*>(gr.pinned);
    MALUS_HIP(hipMemcpyAsync(T(gr.toks)->data(), ids, gr.n * sizeof(int32_t), hipMemcpyHostToDevice, stream()));
    MALUS_HIP(hipMemcpyAsync(T(gr.tgts)->data(), ids + gr.n, gr.n * sizeof(int32_t), hipMemcpyHostToDevice, stream()));
    MALUS_HIP(hipMemcpyAsync(gr.bc->data(), ids + 2 * gr.n, 2 * sizeof(float), hipMemcpyHostToDevice, stream()));
  }
  const uint64_t seq = enqueue_mark("graph inputs");
  T(gr.toks)->write_seq = T(gr.tgts)->write_seq = seq;
  if (gr.drawn) T(gr.calls)->write_seq = seq;
  else gr.bc->write_seq = seq;
  malus_gpt_zero_grad(&g);
  int64_t loss = gpt_forward_loss(g, gr.toks, gr.tgts, nullptr);
  backward(loss);
  adamw_range(g, 0, 8 * g.L + 4, t);
  return loss;
}

// Launches the replay of the inputs just set; returns the loss handle (a
// new reference).
int64_t graph_launch(GptGraph& gr) {
  MALUS_HIP(hipGraphLaunch(gr.exec, stream()));
  MALUS_HIP(hipEventRecord(gr.done, stream()));
  gr.launched = true;
  const uint64_t seq = enqueue_mark("graph step");
  Gpt& g = *gr.g;
  for (size_t i = 0; i < g.p.size(); ++i) T(g.p[i])->write_seq = T(g.m[i])->write_seq = T(g.v[i])->write_seq = seq;
  T(gr.loss)->write_seq = seq;
  tensor_retain(gr.loss);
  return gr.loss;
}

// Releases what a graph holds (any part may still be unset) and detaches
// it from its model.  `prev_inplace` is the model's update mode to restore.
void graph_destroy(GptGraph* gr, bool prev_inplace) {
  (void)hipStreamSynchronize(stream());
  if (gr->exec) (void)hipGraphExecDestroy(gr->exec);
  if (gr->graph) (void)hipGraphDestroy(gr->graph);
  if (gr->done) (void)hipEventDestroy(gr->done);
  if (gr->pinned) (void)hipHostFree(gr->pinned);
  if (gr->loss) tensor_release(gr->loss);
  if (gr->toks) tensor_release(gr->toks);
  if (gr->tgts) tensor_release(gr->tgts);
  if (gr->calls) tensor_release(gr->calls);
  if (gr->bc) release(gr->bc);
  if (gr->g) {
    gr->g->bc_dev = nullptr;
    gr->g->inplace_opt = prev_inplace;
  }
  pool_release_graph(gr->id);
  delete gr;
}

GptGraph* graph_create(Gpt* g, bool drawn, const int32_t* x, const int32_t* y, uint64_t cx, uint64_t cy, int64_t t,
                       int64_t* loss_out) {
  if (g->bc_dev) fail("malus: gpt_graph_create: the model already has a graph");
  const bool prev_inplace = g->inplace_opt;
  auto* gr = new GptGraph();
  gr->id = ++g_graph_ids;
  gr->n = (size_t)g->B * g->Tn;
  gr->drawn = drawn;
  int64_t eager_loss = 0;
  try {
    MALUS_HIP(hipHostMalloc(reinterpret_cast<void**>(&gr->pinned), pinned_bytes(*gr), hipHostMallocDefault));
    const size_t sh[1] = {gr->n}, sh2[1] = {2}, sh3[1] = {3};
    gr->toks = H(alloc_tensor(I32, sh, 1));
    gr->tgts = H(alloc_tensor(I32, sh, 1));
    float* bc_dev;
    if (drawn) {  // the bias corrections share the calls' copy: the two f32 in its third word
      gr->calls = H(alloc_tensor(I64, sh3, 1));
      bc_dev = reinterpret_cast<float*>(static_cast<uint64_t*>(T(gr->calls)->data()) + 2);
    } else {
      gr->bc = alloc_tensor(F32, sh2, 1);
      bc_dev = gr->bc->f32();
    }
    MALUS_HIP(hipEventCreateWithFlags(&gr->done, hipEventDisableTiming));
    gr->g = g;
    g->inplace_opt = true;
    g->bc_dev = bc_dev;
    // eager step t
    graph_set_inputs(*gr, x, y, cx, cy, t);
    eager_loss = graph_step_body(*gr, t);
    MALUS_HIP(hipEventRecord(gr->done, stream()));
    gr->launched = true;
    // capture one step (recorded, not run)
    pool_capture_begin(gr->id);
    MALUS_HIP(hipStreamBeginCapture(stream(), hipStreamCaptureModeRelaxed));
    int64_t cap_loss = 0;
    try {
      cap_loss = graph_step_body(*gr, t + 1);
    } catch (...) {
      hipGraph_t broken = nullptr;
      (void)hipStreamEndCapture(stream(), &broken);
      if (broken) (void)hipGraphDestroy(broken);
      pool_capture_end(gr->id);
      throw;
    }
    MALUS_HIP(hipStreamEndCapture(stream(), &gr->graph));
    pool_capture_end(gr->id);
    gr->loss = cap_loss;
    MALUS_HIP(hipGraphInstantiate(&gr->exec, gr->graph, nullptr, nullptr, 0));
  } catch (...) {
    // The eager step may have run: its in-place update stands (as any
    // eager step's would), and later eager steps use their own bias
    // corrections again.
    if (eager_loss) tensor_release(eager_loss);
    tape_clear();  // the records of a step cut short
    graph_destroy(gr, prev_inplace);
    throw;
  }
  if (loss_out) *loss_out = eager_loss;
  else tensor_release(eager_loss);
  return gr;
}

}  // namespace

extern "C" {

// Runs step t eagerly through the graph's input buffers (it warms the pool
// and returns that step's loss in *loss_out), then captures the step.  The
// model switches to in-place parameter updates; free the graph before the
// model, and leave the tape alone while the graph exists.
void* malus_gpt_graph_create(void* gp, const int32_t* x, const int32_t* y, int64_t t, int64_t* loss_out) {
  API_TRY
  auto* g = static_cast<Gpt*>(gp);
  if (!g || !x || !y) fail("malus: gpt_graph_create: null model or token ids");
  return graph_create(g, false, x, y, 0, 0, t, loss_out);
  API_CATCH(nullptr)
}

// The same with each step's token and target ids drawn on the device by the
// step's own kernel node: x[i] = rand_int(V) with call index x_call + i, y[i]
// with y_call + i (the ids malus_rand_tokens_device returns).
void* malus_gpt_graph_create_drawn(void* gp, uint64_t x_call, uint64_t y_call, int64_t t, int64_t* loss_out) {
  API_TRY
  auto* g = static_cast<Gpt*>(gp);
  if (!g) fail("malus: gpt_graph_create_drawn: null model");
  return graph_create(g, true, nullptr, nullptr, x_call, y_call, t, loss_out);
  API_CATCH(nullptr)
}

// One replay: step t on the given token and target ids.  Returns the loss
// tensor (the same device buffer every step; a new reference the caller
// releases).  Nothing is read back to the host.
int64_t malus_gpt_graph_step(void* gh, const int32_t* x, const int32_t* y, int64_t t) {
  API_TRY
  auto* gr = static_cast<GptGraph*>(gh);
  if (!gr || !x || !y) fail("malus: gpt_graph_step: null graph or token ids");
  if (gr->drawn) fail("malus: gpt_graph_step: this graph draws its ids (use malus_gpt_graph_step_drawn)");
  graph_set_inputs(*gr, x, y, 0, 0, t);
  return graph_launch(*gr);
  API_CATCH(0)
}

// One replay of a graph made by malus_gpt_graph_create_drawn: step t on the
// ids drawn from call indices x_call and y_call.
int64_t malus_gpt_graph_step_drawn(void* gh, uint64_t x_call, uint64_t y_call, int64_t t) {
  API_TRY
  auto* gr = static_cast<GptGraph*>(gh);
  if (!gr) fail("malus: gpt_graph_step_drawn: null graph");
  if (!gr->drawn) fail("malus: gpt_graph_step_drawn: this graph copies its ids (use malus_gpt_graph_step)");
  graph_set_inputs(*gr, nullptr, nullptr, x_call, y_call, t);
  return graph_launch(*gr);
  API_CATCH(0)
}

void malus_gpt_graph_free(void* gh) {
  API_TRY
  auto* gr = static_cast<GptGraph*>(gh);
  if (!gr) return;
  MALUS_HIP(hipStreamSynchronize(stream()));
  graph_destroy(gr, true);  // the model keeps its in-place updates
  API_CATCH()
}

// Kernel nodes of the captured step (the launches one replay stands for).
size_t malus_gpt_graph_nodes(void* gh) {
  auto* gr = static_cast<GptGraph*>(gh);
  size_t n = 0;
  if (gr && gr->graph) MALUS_HIP(hipGraphGetNodes(gr->graph, nullptr, &n));
  return n;
}

// ---- checkpoints (SafeTensors) ------------------------------------------------
// The model's parameters and AdamW moments in the SafeTensors layout: an
// 8-byte little-endian header length, a JSON header (name -> dtype, shape,
// data_offsets; "__metadata__" holds the step and the configuration), then
// the raw little-endian f32 data in header order.  Names follow the program's
// structure: blocks.<l>.{ln1_w,wq,wk,wv,wo,ln2_w,w1,w2}, wte, wpe, ln_f,
// lm_head, and adam_m.<name> / adam_v.<name> for the moments.

}  // extern "C"

namespace {

const char* const kBlockNames[8] = {"ln1_w", "wq", "wk", "wv", "wo", "ln2_w", "w1", "w2"};
const char* const kTopNames[4] = {"wte", "wpe", "ln_f", "lm_head"};

std::string param_name(const Gpt& g, int i) {
  if (i < 8 * g.L) return "blocks." + std::to_string(i / 8) + "." + kBlockNames[i % 8];
  return kTopNames[i - 8 * g.L];
}

// A minimal JSON reader for SafeTensors headers: objects, arrays, strings,
// integers (the values a header holds).
struct Json {
  enum K { Null, Num, Str, Arr, Obj } k = Null;
  long long num = 0;
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;
  const Json* get(const std::string& key) const {
    for (auto& kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

struct JsonParser {
  const std::string& s;
  size_t p = 0;
  [[noreturn]] void bad() { fail("malus: checkpoint header is not valid JSON (at byte %zu)", p); }
  void ws() { while (p < s.size() && isspace((unsigned char)s[p])) ++p; }
  Json value() {
    ws();
    if (p >= s.size()) bad();
    Json j;
    if (s[p] == '{') {
      j.k = Json::Obj;
      ++p;
      ws();
      if (p < s.size() && s[p] == '}') { ++p; return j; }
      while (true) {
        ws();
        Json key = value();
        if (key.k != Json::Str) bad();
        ws();
        if (p >= s.size() || s[p] != ':') bad();
        ++p;
        j.obj.emplace_back(key.str, value());
        ws();
        if (p < s.size() && s[p] == ',') { ++p; continue; }
        if (p < s.size() && s[p] == '}') { ++p; return j; }
        bad();
      }
    }
    if (s[p] == '[') {
      j.k = Json::Arr;
      ++p;
      ws();
      if (p < s.size() && s[p] == ']') { ++p; return j; }
      while (true) {
        j.arr.push_back(value());
        ws();
        if (p < s.size() && s[p] == ',') { ++p; continue; }
        if (p < s.size() && s[p] == ']') { ++p; return j; }
        bad();
      }
    }
    if (s[p] == '"') {
      j.k = Json::Str;
      ++p;
      while (p < s.size() && s[p] != '"') {
        if (s[p] == '\\' && p + 1 < s.size()) ++p;
        j.str += s[p++];
      }
      if (p >= s.size()) bad();
      ++p;
      return j;
    }
    if (s[p] == '-' || isdigit((unsigned char)s[p])) {
      j.k = Json::Num;
      size_t e = p + 1;
      while (e < s.size() && (isdigit((unsigned char)s[e]) || s[e] == '.' || s[e] == 'e' || s[e] == 'E' ||
                              s[e] == '+' || s[e] == '-'))
        ++e;
      j.num = strtoll(s.c_str() + p, nullptr, 10);
      p = e;
      return j;
    }
    if (s.compare(p, 4, "null") == 0) { p += 4; return j; }
    if (s.compare(p, 4, "true") == 0) { p += 4; j.k = Json::Num; j.num = 1; return j; }
    if (s.compare(p, 5, "false") == 0) { p += 5; j.k = Json::Num; return j; }
    bad();
  }
};

}  // namespace

extern "C" {

// Writes the model (parameters and moments) and `step` to `path`.
// Returns 0, or -1 in return-error mode.
int malus_gpt_save(void* gp, const char* path, int64_t step) {
  API_TRY
  auto* g = static_cast<Gpt*>(gp);
  if (!g || !path) fail("malus: gpt_save: null model or path");
  struct Item { std::string name; int64_t h; };
  std::vector<Item> items;
  for (int i = 0; i < g->np(); ++i) items.push_back({param_name(*g, i), g->p[(size_t)i]});
  for (int i = 0; i < g->np(); ++i) items.push_back({"adam_m." + param_name(*g, i), g->m[(size_t)i]});
  for (int i = 0; i < g->np(); ++i) items.push_back({"adam_v." + param_name(*g, i), g->v[(size_t)i]});
  std::string hdr = "{\"__metadata__\":{\"format\":\"malus\",\"step\":\"" + std::to_string(step) + "\",\"config\":\"V=" +
                    std::to_string(g->V) + ",T=" + std::to_string(g->Tn) + ",C=" + std::to_string(g->C) + ",H=" +
                    std::to_string(g->H) + ",L=" + std::to_string(g->L) + "\"}";
  size_t off = 0;
  for (auto& it : items) {
    TensorBuffer* t = T(it.h);
    hdr += ",\"" + it.name + "\":{\"dtype\":\"F32\",\"shape\":[";
    for (int d = 0; d < t->ndim; ++d) hdr += (d ? "," : "") + std::to_string(t->shape[d]);
    hdr += "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(off + t->bytes()) + "]}";
    off += t->bytes();
  }
  hdr += "}";
  while (hdr.size() % 8) hdr += ' ';
  FILE* f = fopen(path, "wb");
  if (!f) fail("malus: gpt_save: cannot open %s for writing", path);
  uint64_t n = hdr.size();
  unsigned char len[8];
  for (int b = 0; b < 8; ++b) len[b] = (unsigned char)(n >> (8 * b));
  bool ok = fwrite(len, 1, 8, f) == 8 && fwrite(hdr.data(), 1, hdr.size(), f) == hdr.size();
  std::vector<char> buf;
  for (auto& it : items) {
    TensorBuffer* t = T(it.h);
    buf.resize(t->bytes());
    download(buf.data(), t, t->bytes());
    ok = ok && fwrite(buf.data(), 1, buf.size(), f) == buf.size();
  }
  ok = (fclose(f) == 0) && ok;
  if (!ok) fail("malus: gpt_save: write to %s failed", path);
  return 0;
  API_CATCH(-1)
}

// Reads parameters and moments from `path` into the model (names, dtypes and
// shapes must match) and returns the stored step (-1 in return-error mode).
int64_t malus_gpt_load(void* gp, const char* path) {
  API_TRY
  auto* g = static_cast<Gpt*>(gp);
  if (!g || !path) fail("malus: gpt_load: null model or path");
  FILE* f = fopen(path, "rb");
  if (!f) fail("malus: gpt_load: cannot open %s", path);
  unsigned char len[8];
  if (fread(len, 1, 8, f) != 8) { fclose(f); fail("malus: gpt_load: %s is too short", path); }
  uint64_t n = 0;
  for (int b = 0; b < 8; ++b) n |= (uint64_t)len[b] << (8 * b);
  if (n > (uint64_t)1 << 30) { fclose(f); fail("malus: gpt_load: header of %llu bytes", (unsigned long long)n); }
  std::string hdr(n, '\0');
  if (fread(&hdr[0], 1, n, f) != n) { fclose(f); fail("malus: gpt_load: truncated header in %s", path); }
  fseek(f, 0, SEEK_END);
  const long total = ftell(f);
  const uint64_t data0 = 8 + n;
  Json root;
  try {
    JsonParser jp{hdr};
    root = jp.value();
  } catch (...) {
    fclose(f);
    throw;
  }
  // Every entry is checked before any is read: F32, the model's shape, and
  // data offsets [begin, end) with 0 <= begin <= end <= the data section's
  // size, end - begin = the tensor's bytes, and no two ranges overlapping.
  struct Item {
    int64_t h;
    uint64_t begin, end;
    std::string name;
  };
  std::vector<Item> items;
  auto check_one = [&](const std::string& name, int64_t h) {
    const Json* e = root.get(name);
    if (!e) fail("malus: gpt_load: %s has no tensor named %s", path, name.c_str());
    const Json* dt = e->get("dtype");
    const Json* sh = e->get("shape");
    const Json* of = e->get("data_offsets");
    if (!dt || dt->str != "F32") fail("malus: gpt_load: %s is not F32", name.c_str());
    TensorBuffer* t = T(h);
    if (!sh || sh->k != Json::Arr || (int)sh->arr.size() != t->ndim) fail("malus: gpt_load: %s has the wrong rank", name.c_str());
    for (int d = 0; d < t->ndim; ++d)
      if (sh->arr[(size_t)d].k != Json::Num || sh->arr[(size_t)d].num < 0 ||
          (size_t)sh->arr[(size_t)d].num != t->shape[d])
        fail("malus: gpt_load: %s has shape mismatching the model's %s", name.c_str(), shape_str(t).c_str());
    if (!of || of->k != Json::Arr || of->arr.size() != 2 || of->arr[0].k != Json::Num || of->arr[1].k != Json::Num)
      fail("malus: gpt_load: %s has no [begin, end] data offsets", name.c_str());
    const long long b0 = of->arr[0].num, e0 = of->arr[1].num;
    const uint64_t data_bytes = (uint64_t)total > data0 ? (uint64_t)total - data0 : 0;
    if (b0 < 0 || e0 < b0 || (uint64_t)e0 > data_bytes || (uint64_t)(e0 - b0) != t->bytes())
      fail("malus: gpt_load: %s has bad data offsets [%lld, %lld) for %zu bytes in a %llu-byte data section",
           name.c_str(), b0, e0, t->bytes(), (unsigned long long)data_bytes);
    items.push_back({h, (uint64_t)b0, (uint64_t)e0, name});
  };
  try {
    for (int i = 0; i < g->np(); ++i) {
      check_one(param_name(*g, i), g->p[(size_t)i]);
      check_one("adam_m." + param_name(*g, i), g->m[(size_t)i]);
      check_one("adam_v." + param_name(*g, i), g->v[(size_t)i]);
    }
    std::vector<const Item*> order;
    for (auto& it : items) order.push_back(&it);
    std::sort(order.begin(), order.end(), [](const Item* x, const Item* y) { return x->begin < y->begin; });
    for (size_t i = 1; i < order.size(); ++i)
      if (order[i]->begin < order[i - 1]->end)
        fail("malus: gpt_load: the data of %s and %s overlap", order[i - 1]->name.c_str(), order[i]->name.c_str());
    for (auto& it : items) {
      TensorBuffer* t = T(it.h);
      std::vector<char> buf(t->bytes());
      fseek(f, (long)(data0 + it.begin), SEEK_SET);
      if (fread(buf.data(), 1, buf.size(), f) != buf.size()) fail("malus: gpt_load: short read of %s", it.name.c_str());
      upload(t->data(), buf.data(), buf.size());
      t->write_seq = enqueue_mark("checkpoint load");
    }
  } catch (...) {
    fclose(f);
    throw;
  }
  fclose(f);
  int64_t step = 0;
  if (const Json* md = root.get("__metadata__"))
    if (const Json* st = md->get("step")) step = strtoll(st->str.c_str(), nullptr, 10);
  return step;
  API_CATCH(-1)
}

}  // extern "C"
