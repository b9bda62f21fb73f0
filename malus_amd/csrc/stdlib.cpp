// Stdlib host functions: the operations malus `fn` bodies dispatch
// implicitly (crates/malus-stdlib/stdlib/*.ml and backward/*.ml), each
// implemented on the hand-written gfx950 kernels with its own launch
// geometry.  Names mirror the .ml host fns with a malus_std_ prefix; the
// backward ones are what the tape's BwdSlot table holds by default.
//
// Where the .ml composition launches several kernels (softmax VJP: 5,
// layernorm VJP: ~10, cross-entropy: 3, AdamW: ~16 per tensor) one fused
// kernel computes the same f32 expression tree.  Output handles are owned
// by the caller (refcount 1); inputs are borrowed.
#include <cmath>
#include <cstring>
#include <vector>

#include "api.h"
#include "common.h"

using namespace malus;

namespace {

int norm_axis(int64_t axis, int ndim) {
  int64_t a = axis < 0 ? axis + ndim : axis;  // normalize_axis, metal.rs:1124-1131
  if (a < 0 || a >= ndim) fail("malus: axis %lld is out of range for tensor with %d dimensions", (long long)axis, ndim);
  return (int)a;
}

void split_axis(const TensorBuffer* t, int axis, size_t* outer, size_t* a, size_t* inner) {
  size_t o = 1, in = 1;
  for (int i = 0; i < axis; ++i) o *= t->shape[i];
  for (int i = axis + 1; i < t->ndim; ++i) in *= t->shape[i];
  *outer = o;
  *a = t->shape[axis];
  *inner = in;
}

void need_f32(const TensorBuffer* t, const char* what) {
  if (t->dtype != F32) fail("malus: %s expects a Tensor<f32>, got dtype tag %d", what, t->dtype);
}

// GEMM operands may be f32 or bf16 (the autocast activations); the mask of
// bf16-stored operands for GemmLayouts::io.
int gemm_io(const TensorBuffer* a, const TensorBuffer* b, const char* what) {
  for (const TensorBuffer* t : {a, b})
    if (t->dtype != F32 && t->dtype != BF16)
      fail("malus: %s expects Tensor<f32> or Tensor<bf16> operands, got dtype tag %d", what, t->dtype);
  if (a->split3) fail("malus: %s: a split copy is read only as B", what);
  return (a->dtype == BF16 ? k::kIoA16 : 0) | (b->split3 ? k::kIoB3 : b->dtype == BF16 ? k::kIoB16 : 0);
}

// The tensor a GEMM reads for operand t: t's copy when it holds t's
// current values (refreshed after t's last write).  Under autocast that is
// t's bf16 copy (the bf16 MFMA rounds t to those values anyway).  With
// split f32 products it is t's split copy (the pieces the product would
// split t into, so the same bits), for the B operand of a GEMM with neither
// operand transposed (split_b: the forward products; on the NT dx products
// the three planes measured slower than splitting the weight in place).
const TensorBuffer* gemm_operand(const TensorBuffer* t, bool split_b = false) {
  const TensorBuffer* c = t->bf16_copy;
  if (!c || c->copy_of != t || c->copy_seq != t->write_seq) return t;
  if (c->split3) return split_b && !k::autocast_on() && k::gemm_f32_split() ? c : t;
  return k::autocast_on() ? c : t;
}

int64_t done(TensorBuffer* t, const char* name) {
  t->write_seq = enqueue_mark(name);
  return H(t);
}

bool same_shape(const TensorBuffer* a, const TensorBuffer* b) {
  if (a->ndim != b->ndim) return false;
  for (int i = 0; i < a->ndim; ++i)
    if (a->shape[i] != b->shape[i]) return false;
  return true;
}

TensorBuffer* copy_of(const TensorBuffer* t) {
  TensorBuffer* o = alloc_like(t);
  k::copy(t->data(), o->data(), t->bytes(), stream());
  o->write_seq = enqueue_mark("copy");
  return o;
}

// p op q with NumPy right-aligned broadcasting; p has rank >= q's rank.
TensorBuffer* broadcast_binop(int op, const TensorBuffer* p, const TensorBuffer* q) {
  const int n = p->ndim;
  size_t qq[kMaxRank], os[kMaxRank];
  for (int i = 0; i < n; ++i) {
    qq[i] = i >= n - q->ndim ? q->shape[i - (n - q->ndim)] : 1;
    size_t pd = p->shape[i];
    if (pd == qq[i] || qq[i] == 1) os[i] = pd;
    else if (pd == 1) os[i] = qq[i];
    else
      fail("malus: broadcast shape mismatch at dim %d: %zu vs %zu\n  left shape:  %s\n  right shape: %s", i, pd, qq[i],
           shape_str(p).c_str(), shape_str(q).c_str());
  }
  TensorBuffer* out = alloc_tensor(F32, os, n);
  hipStream_t s = stream();
  const size_t total = out->len;
  bool out_is_p = true;
  for (int i = 0; i < n; ++i) out_is_p &= (os[i] == p->shape[i]);
  if (out_is_p && q->len == p->len) {
    k::binary_same(op, p->f32(), q->f32(), out->f32(), total, s);
  } else if (out_is_p && q->len == 1) {
    k::binary_scalar(op, p->f32(), q->f32(), 0.0f, true, out->f32(), total, s);
  } else {
    // q is a trailing block of p: q's padded shape = [1.., p.shape[k..]]
    bool trailing = out_is_p;
    if (trailing) {
      int k0 = 0;
      while (k0 < n && qq[k0] == 1) ++k0;
      for (int i = k0; i < n; ++i) trailing &= (qq[i] == p->shape[i]);
    }
    if (trailing && total % q->len == 0) {
      k::binary_rowbcast(op, p->f32(), q->f32(), out->f32(), total, q->len, s);
    } else {
      k::BcastDesc d{};
      d.ndim = n;
      size_t ps = 1, qs = 1;
      for (int i = n - 1; i >= 0; --i) {
        d.out_shape[i] = (uint32_t)os[i];
        d.p_stride[i] = p->shape[i] == 1 ? 0u : (uint32_t)ps;
        d.q_stride[i] = qq[i] == 1 ? 0u : (uint32_t)qs;
        ps *= p->shape[i];
        qs *= qq[i];
      }
      k::binary_general(op, p->f32(), q->f32(), out->f32(), total, d, s);
    }
  }
  return out;
}

// Reduce `dout` down to `target`'s shape (sum over broadcast dims),
// elementwise_bwd.ml:8-22.  Equal shapes return a retained alias.  With
// `mul` (same shape as g), reduces g * mul without materializing it: the
// first reduction pass multiplies on load, every product rounded to f32 as
// the materialized tensor's would be, so results are bit-identical.
TensorBuffer* sum_to_shape(TensorBuffer* g, const TensorBuffer* target, const TensorBuffer* mul = nullptr) {
  if (same_shape(g, target)) {
    if (!mul) {
      retain(g);
      return g;
    }
    TensorBuffer* out = alloc_tensor(F32, target->shape, target->ndim);
    k::binary_same(k::MUL, g->f32(), mul->f32(), out->f32(), out->len, stream());
    return out;
  }
  const int gn = g->ndim, tn = target->ndim;
  if (tn > gn) fail("malus: sum_to_shape: target rank %d exceeds gradient rank %d", tn, gn);
  size_t padded[kMaxRank];
  for (int i = 0; i < gn; ++i) padded[i] = i >= gn - tn ? target->shape[i - (gn - tn)] : 1;
  for (int i = 0; i < gn; ++i)
    if (padded[i] != 1 && padded[i] != g->shape[i])
      fail("malus: sum_to_shape: %s is not broadcastable to %s", shape_str(target).c_str(), shape_str(g).c_str());
  // classify dims: reduce (padded 1, g > 1) or keep; merge runs
  struct Run { bool red; size_t n; };
  std::vector<Run> runs;
  for (int i = 0; i < gn; ++i) {
    bool red = padded[i] == 1 && g->shape[i] != 1;
    size_t n = g->shape[i];
    if (n == 1) continue;  // size-1 dims are layout-neutral
    if (!runs.empty() && runs.back().red == red) runs.back().n *= n;
    else runs.push_back({red, n});
  }
  TensorBuffer* out = alloc_tensor(F32, target->shape, tn);
  hipStream_t s = stream();
  // reduce runs one at a time from the last, keeping a running [.., R, K] view
  const float* src = g->f32();
  const float* src_mul = mul ? mul->f32() : nullptr;  // applies to the first pass only
  std::vector<std::pair<void*, size_t>> temps;
  size_t cur_len = g->len;
  for (int r = (int)runs.size() - 1; r >= 0; --r) {
    if (!runs[r].red) continue;
    size_t inner = 1, outer = 1;
    for (size_t j = r + 1; j < runs.size(); ++j) inner *= runs[j].n;
    outer = cur_len / (runs[r].n * inner);
    size_t out_len = outer * inner;
    bool last = true;
    for (int j = r - 1; j >= 0; --j) last &= !runs[j].red;
    float* dst;
    if (last) {
      dst = out->f32();
    } else {
      size_t b;
      dst = static_cast<float*>(pool_alloc(out_len * sizeof(float), &b));
      temps.push_back({dst, b});
    }
    if (src_mul) k::reduce_axis_prod(src, src_mul, dst, outer, runs[r].n, inner, s);
    else k::reduce_axis(k::R_SUM, src, dst, outer, runs[r].n, inner, s);
    src_mul = nullptr;
    src = dst;
    cur_len = out_len;
    runs[r].n = 1;
  }
  if (src != out->f32()) {  // nothing to reduce (all size-1)
    if (src_mul) k::binary_same(k::MUL, src, src_mul, out->f32(), out->len, s);
    else k::copy(src, out->f32(), out->bytes(), s);
  }
  for (auto& t : temps) pool_free(t.first, t.second);
  return out;
}

// [outer, a, inner] broadcast of a keepdim/non-keepdim reduced tensor
TensorBuffer* expand_to(const TensorBuffer* small, const TensorBuffer* tmpl, int axis) {
  size_t o, a, in;
  split_axis(tmpl, axis, &o, &a, &in);
  if (small->len != o * in)
    fail("malus: expand_axis: small tensor %s does not match %s reduced over axis %d", shape_str(small).c_str(),
         shape_str(tmpl).c_str(), axis);
  TensorBuffer* out = alloc_tensor(F32, tmpl->shape, tmpl->ndim);
  k::expand_axis(small->f32(), out->f32(), o, a, in, stream());
  return out;
}

TensorBuffer* as_i32_indices(TensorBuffer* idx, bool* owned) {
  *owned = false;
  if (idx->dtype == I32) return idx;
  fail("malus: index tensors must be Tensor<i32> (got dtype tag %d)", idx->dtype);
}

int64_t gemm_out(const TensorBuffer* a, const TensorBuffer* b, bool ta, bool tb, int batch, int M, int N, int K, long sA,
                 long sB, const size_t* oshape, int ond, const TensorBuffer* addend = nullptr) {
  a = gemm_operand(a);
  b = gemm_operand(b, !ta && !tb);
  const int io = gemm_io(a, b, "matmul");
  TensorBuffer* c = alloc_tensor(F32, oshape, ond);
  if (addend && (addend->dtype != F32 || addend->len != c->len))
    fail("malus: matmul accumulate: addend %s does not match the product %s", shape_str(addend).c_str(), shape_str(c).c_str());
  KTimer* kt = ktimer_begin("gemm");
  k::gemm(a->f32(), b->f32(), c->f32(), batch, M, N, K, ta, tb, sA, sB, (long)M * N, stream(),
          addend ? addend->f32() : nullptr, io);
  ktimer_end(kt, 2.0 * batch * (double)M * N * K);
  return done(c, "matmul");
}

}  // namespace

extern "C" {

// ---- broadcast binops (broadcast_binop.ml:82-112, operand swap kept) -------
int64_t malus_std_broadcast_fwd(int32_t op, int64_t a, int64_t b) {
  API_TRY
  TensorBuffer *ta = T(a), *tb = T(b);
  need_f32(ta, "broadcast op");
  need_f32(tb, "broadcast op");
  TensorBuffer* out = ta->ndim >= tb->ndim ? broadcast_binop(op, ta, tb) : broadcast_binop(op, tb, ta);
  return done(out, "broadcast");
  API_CATCH(0)
}
int64_t malus_std_broadcast_add_fwd(int64_t a, int64_t b) { return malus_std_broadcast_fwd(k::ADD, a, b); }
int64_t malus_std_broadcast_sub_fwd(int64_t a, int64_t b) { return malus_std_broadcast_fwd(k::SUB, a, b); }
int64_t malus_std_broadcast_mul_fwd(int64_t a, int64_t b) { return malus_std_broadcast_fwd(k::MUL, a, b); }
int64_t malus_std_broadcast_div_fwd(int64_t a, int64_t b) { return malus_std_broadcast_fwd(k::DIV, a, b); }

// ---- scalar builtins (codegen-gpu/lib.rs:400-418) ---------------------------
int64_t malus_std_scalar_op(int32_t op, int64_t a, float s, int32_t right) {
  API_TRY
  TensorBuffer* t = T(a);
  need_f32(t, "scalar op");
  TensorBuffer* out = alloc_like(t);
  k::binary_scalar(op, t->f32(), nullptr, s, right != 0, out->f32(), t->len, stream());
  return done(out, "scalar_op");
  API_CATCH(0)
}
int64_t malus_std_scalar_op_dev(int32_t op, int64_t a, int64_t s1, int32_t right) {
  API_TRY
  TensorBuffer *t = T(a), *sv = T(s1);
  need_f32(t, "scalar op");
  if (sv->len < 1) fail("malus: scalar operand tensor is empty");
  TensorBuffer* out = alloc_like(t);
  k::binary_scalar(op, t->f32(), sv->f32(), 0.0f, right != 0, out->f32(), t->len, stream());
  return done(out, "scalar_op");
  API_CATCH(0)
}

// ---- unary builtins (codegen-gpu/lib.rs:375-381) ---------------------------
int64_t malus_std_unary(int32_t op, int64_t x) {
  API_TRY
  TensorBuffer* t = T(x);
  need_f32(t, "unary op");
  TensorBuffer* out = alloc_like(t);
  k::unary(op, t->f32(), out->f32(), t->len, stream());
  return done(out, "unary");
  API_CATCH(0)
}
int64_t malus_std_gelu_fwd(int64_t x) { return malus_std_unary(k::GELU, x); }

// The stdlib's f32 <-> bf16 conversion (docs/adr/0037-bf16-autocast.md:30,
// "conversion kernels (f32<->bf16) join the stdlib"): a new tensor of the
// same shape in `dtype` (F32 or BF16); to bf16 rounds to nearest even, to
// f32 is exact; a same-dtype cast copies.
int64_t malus_std_cast(int64_t x, int32_t dtype) {
  API_TRY
  TensorBuffer* t = T(x);
  if ((t->dtype != F32 && t->dtype != BF16) || (dtype != F32 && dtype != BF16))
    fail("malus: cast supports f32 and bf16 only (dtype tags %d -> %d)", t->dtype, dtype);
  TensorBuffer* out = alloc_tensor(dtype, t->shape, t->ndim);
  if (t->dtype == dtype) k::copy(t->data(), out->data(), t->bytes(), stream());
  else k::convert_f32_bf16(t->data(), out->data(), t->len, dtype == BF16, stream());
  return done(out, "cast");
  API_CATCH(0)
}

// ---- axis reductions (reduce_{sum,mean,max,var}.ml) ------------------------
int64_t malus_std_reduce_fwd(int32_t op, int64_t x, int64_t axis, int64_t keepdim) {
  API_TRY
  TensorBuffer* t = T(x);
  need_f32(t, "reduction");
  int ax = norm_axis(axis, t->ndim);
  size_t o, a, in;
  split_axis(t, ax, &o, &a, &in);
  size_t sh[kMaxRank];
  int nd = 0;
  if (t->ndim == 1) {
    sh[nd++] = 1;  // reduce_sum.ml:32-33: rank-1 input -> [1]
  } else {
    for (int i = 0; i < t->ndim; ++i) {
      if (i == ax) { if (keepdim) sh[nd++] = 1; }
      else sh[nd++] = t->shape[i];
    }
  }
  TensorBuffer* out = alloc_tensor(F32, sh, nd);
  k::reduce_axis(op, t->f32(), out->f32(), o, a, in, stream());
  return done(out, "reduce");
  API_CATCH(0)
}

// reduce_all.ml:9-12: whole-tensor sum -> [1] (no 1024-element cap here)
int64_t malus_std_reduce_all_sum_fwd(int64_t x) {
  API_TRY
  TensorBuffer* t = T(x);
  need_f32(t, "sum");
  TensorBuffer* out = alloc_f32({1});
  k::reduce_axis(k::R_SUM, t->f32(), out->f32(), 1, t->len, 1, stream());
  return done(out, "sum_all");
  API_CATCH(0)
}

// ---- softmax / layernorm / cross-entropy ------------------------------------
int64_t malus_std_softmax_fwd(int64_t x, int64_t axis) {
  API_TRY
  TensorBuffer* t = T(x);
  need_f32(t, "softmax");
  int ax = norm_axis(axis, t->ndim);
  size_t o, a, in;
  split_axis(t, ax, &o, &a, &in);
  TensorBuffer* out = alloc_like(t);
  k::softmax(t->f32(), out->f32(), o, a, in, stream());
  return done(out, "softmax");
  API_CATCH(0)
}

// Returns normed; *var_out receives the population variance, keepdim at the
// axis (the tape takes ownership, tape.rs:289-310).
int64_t malus_std_layernorm_fwd(int64_t x, int64_t axis, int64_t* var_out) {
  API_TRY
  TensorBuffer* t = T(x);
  need_f32(t, "layernorm");
  int ax = norm_axis(axis, t->ndim);
  size_t o, a, in;
  split_axis(t, ax, &o, &a, &in);
  TensorBuffer* y = alloc_like(t);
  size_t vsh[kMaxRank];
  for (int i = 0; i < t->ndim; ++i) vsh[i] = i == ax ? 1 : t->shape[i];
  TensorBuffer* var = alloc_tensor(F32, vsh, t->ndim);
  k::layernorm(t->f32(), y->f32(), var->f32(), o, a, in, 1e-5f, stream());
  uint64_t seq = enqueue_mark("layernorm");
  y->write_seq = var->write_seq = seq;
  if (var_out) *var_out = H(var);
  else release(var);
  return H(y);
  API_CATCH(0)
}

// cross_entropy.ml:18-28: returns loss [1]; *probs_out receives the softmax
// probabilities [N, V].
int64_t malus_std_cross_entropy_fwd(int64_t logits, int64_t targets, int64_t* probs_out) {
  API_TRY
  TensorBuffer *lg = T(logits), *tg = T(targets);
  need_f32(lg, "cross_entropy");
  if (lg->ndim != 2) fail("malus: cross_entropy logits must be rank-2 [N, C], got shape %s", shape_str(lg).c_str());
  if (tg->ndim != 1) fail("malus: cross_entropy targets must be rank-1 [N], got shape %s", shape_str(tg).c_str());
  const size_t n = lg->shape[0], v = lg->shape[1];
  if (tg->shape[0] != n) fail("malus: cross_entropy logits N=%zu but targets has %zu elements", n, tg->shape[0]);
  bool owned;
  TensorBuffer* ti = as_i32_indices(tg, &owned);
  TensorBuffer* probs = alloc_like(lg);
  TensorBuffer* loss = alloc_f32({1});
  size_t b;
  float* nll = static_cast<float*>(pool_alloc(n * sizeof(float), &b));
  hipStream_t s = stream();
  k::ce_fwd(lg->f32(), ti->i32(), probs->f32(), nll, n, v, device_error_flag(), s);
  k::reduce_axis(k::R_MEAN, nll, loss->f32(), 1, n, 1, s);  // reduce_mean_fwd(nll, 0, 1)
  pool_free(nll, b);
  uint64_t seq = enqueue_mark("cross_entropy");
  probs->write_seq = loss->write_seq = seq;
  if (probs_out) *probs_out = H(probs);
  else release(probs);
  return H(loss);
  API_CATCH(0)
}

// ---- embedding (embedding.ml:18-23) -----------------------------------------
int64_t malus_std_embedding_fwd(int64_t weight, int64_t indices) {
  API_TRY
  TensorBuffer *w = T(weight), *idx = T(indices);
  need_f32(w, "embedding");
  if (w->ndim != 2) fail("malus: embedding weight must be rank-2 [V, D], got shape %s", shape_str(w).c_str());
  if (idx->ndim != 1) fail("malus: embedding indices must be rank-1 [T], got shape %s", shape_str(idx).c_str());
  bool owned;
  TensorBuffer* ii = as_i32_indices(idx, &owned);
  size_t sh[2] = {idx->len, w->shape[1]};
  TensorBuffer* out = alloc_tensor(F32, sh, 2);
  k::embedding(w->f32(), ii->i32(), out->f32(), idx->len, w->shape[0], w->shape[1], device_error_flag(), stream());
  return done(out, "embedding");
  API_CATCH(0)
}

// ---- permutes (permute.ml) ---------------------------------------------------
static int64_t permute_impl(TensorBuffer* t, const std::vector<size_t>& perm) {
  need_f32(t, "permute");
  if ((int)perm.size() != t->ndim) fail("malus: permute of rank %zu for a rank-%d tensor", perm.size(), t->ndim);
  size_t osh[kMaxRank];
  for (int d = 0; d < t->ndim; ++d) osh[d] = t->shape[perm[d]];
  TensorBuffer* out = alloc_tensor(F32, osh, t->ndim);
  k::permute(t->f32(), out->f32(), t->ndim, t->shape, perm.data(), stream());
  return done(out, "permute");
}

int64_t malus_std_transpose_2d_fwd(int64_t x) {
  API_TRY
  TensorBuffer* t = T(x);
  if (t->ndim != 2) fail("malus: transpose requires a 2-D tensor, got shape %s", shape_str(t).c_str());
  return permute_impl(t, {1, 0});
  API_CATCH(0)
}
int64_t malus_std_permute_3d_fwd(int64_t x, int64_t p0, int64_t p1, int64_t p2) {
  API_TRY
  TensorBuffer* t = T(x);
  std::vector<size_t> perm = tape_normalize_perm({(size_t)p0, (size_t)p1, (size_t)p2}, (size_t)t->ndim);
  return permute_impl(t, perm);
  API_CATCH(0)
}
int64_t malus_std_permute_nd_fwd(int64_t x, int64_t p0, int64_t p1, int64_t p2, int64_t p3, int64_t p4, int64_t p5,
                                 int64_t p6, int64_t p7) {
  API_TRY
  TensorBuffer* t = T(x);
  int64_t all[8] = {p0, p1, p2, p3, p4, p5, p6, p7};
  std::vector<size_t> perm;
  for (int i = 0; i < t->ndim; ++i) perm.push_back((size_t)all[i]);
  return permute_impl(t, tape_normalize_perm(perm, (size_t)t->ndim));
  API_CATCH(0)
}

// tensor_permute, metal.rs:1405-1417: normalize, then the PermuteNdFwd slot.
int64_t tensor_permute(int64_t h, const size_t* perm_ptr, size_t n) {
  API_TRY
  TensorBuffer* t = T(h);
  std::vector<size_t> raw;
  if (perm_ptr && n) raw.assign(perm_ptr, perm_ptr + n);
  std::vector<size_t> perm = tape_normalize_perm(raw, (size_t)t->ndim);
  int64_t p[8] = {0};
  for (size_t i = 0; i < perm.size(); ++i) p[i] = (int64_t)perm[i];
  using FnPerm = int64_t (*)(int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t);
  auto f = reinterpret_cast<FnPerm>(malus_tape_backward_fn(17));
  return f(h, p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7]);
  API_CATCH(0)
}

// ---- unary_bwd.ml helpers ------------------------------------------------------
int64_t malus_std_scale_fwd(int64_t x, float c) { return malus_std_scalar_op(k::MUL, x, c, 1); }
int64_t malus_std_fill_like_fwd(int64_t x, float c) {
  API_TRY
  TensorBuffer* t = T(x);
  TensorBuffer* out = alloc_tensor(F32, t->shape, t->ndim);
  k::fill(out->f32(), c, out->len, stream());
  return done(out, "fill_like");
  API_CATCH(0)
}
int64_t malus_std_eq_fwd(int64_t a, int64_t b) {
  API_TRY
  TensorBuffer *ta = T(a), *tb = T(b);
  if (ta->len != tb->len) fail("malus: eq requires equal lengths, got %zu and %zu", ta->len, tb->len);
  TensorBuffer* out = alloc_like(ta);
  k::eq(ta->f32(), tb->f32(), out->f32(), ta->len, stream());
  return done(out, "eq");
  API_CATCH(0)
}
int64_t malus_std_expand_axis_fwd(int64_t small, int64_t x_template, int64_t axis) {
  API_TRY
  TensorBuffer* tmpl = T(x_template);
  return done(expand_to(T(small), tmpl, norm_axis(axis, tmpl->ndim)), "expand_axis");
  API_CATCH(0)
}
int64_t malus_std_sum_to_shape_bwd(int64_t dout, int64_t target) {
  API_TRY
  TensorBuffer* r = sum_to_shape(T(dout), T(target));
  if (r == T(dout)) return H(r);  // retained alias, already complete
  return done(r, "sum_to_shape");
  API_CATCH(0)
}

// ---- elementwise_bwd.ml ------------------------------------------------------
int64_t malus_std_add_bwd_a(int64_t dout, int64_t a) { return malus_std_sum_to_shape_bwd(dout, a); }
int64_t malus_std_add_bwd_b(int64_t dout, int64_t b) { return malus_std_sum_to_shape_bwd(dout, b); }
int64_t malus_std_sub_bwd_a(int64_t dout, int64_t a) { return malus_std_sum_to_shape_bwd(dout, a); }
int64_t malus_std_sub_bwd_b(int64_t dout, int64_t b) {
  API_TRY
  int64_t neg = malus_std_scale_fwd(dout, -1.0f);
  int64_t r = malus_std_sum_to_shape_bwd(neg, b);
  release(T(neg));
  return r;
  API_CATCH(0)
}
int64_t malus_std_mul_bwd_a(int64_t dout, int64_t a, int64_t b) {
  API_TRY
  if (same_shape(T(dout), T(b)) && !same_shape(T(dout), T(a)))  // reduce dout * b without materializing it
    return done(sum_to_shape(T(dout), T(a), T(b)), "mul_bwd_a");
  int64_t full = malus_std_broadcast_mul_fwd(dout, b);
  int64_t r = malus_std_sum_to_shape_bwd(full, a);
  release(T(full));
  return r;
  API_CATCH(0)
}
int64_t malus_std_mul_bwd_b(int64_t dout, int64_t a, int64_t b) {
  API_TRY
  if (same_shape(T(dout), T(a)) && !same_shape(T(dout), T(b)))  // reduce dout * a without materializing it
    return done(sum_to_shape(T(dout), T(b), T(a)), "mul_bwd_b");
  int64_t full = malus_std_broadcast_mul_fwd(dout, a);
  int64_t r = malus_std_sum_to_shape_bwd(full, b);
  release(T(full));
  return r;
  API_CATCH(0)
}
int64_t malus_std_div_bwd_a(int64_t dout, int64_t a, int64_t b) {
  API_TRY
  int64_t full = malus_std_broadcast_div_fwd(dout, b);
  int64_t r = malus_std_sum_to_shape_bwd(full, a);
  release(T(full));
  return r;
  API_CATCH(0)
}
int64_t malus_std_div_bwd_b(int64_t dout, int64_t a, int64_t b) {
  API_TRY
  int64_t t1 = malus_std_broadcast_mul_fwd(dout, a);
  int64_t neg = malus_std_scale_fwd(t1, -1.0f);
  int64_t bsq = malus_std_broadcast_mul_fwd(b, b);
  int64_t full = malus_std_broadcast_div_fwd(neg, bsq);
  int64_t r = malus_std_sum_to_shape_bwd(full, b);
  release(T(t1)); release(T(neg)); release(T(bsq)); release(T(full));
  return r;
  API_CATCH(0)
}

// ---- unary VJPs (unary_bwd.ml:37-91) -------------------------------------------
static int64_t unary_bwd_impl(int op, int64_t xy, int64_t dout) {
  TensorBuffer *a = T(xy), *d = T(dout);
  if (a->len != d->len) fail("malus: unary VJP length mismatch %zu vs %zu", a->len, d->len);
  TensorBuffer* out = alloc_like(a);
  k::unary_bwd(op, a->f32(), d->f32(), out->f32(), a->len, stream());
  return done(out, "unary_bwd");
}
int64_t malus_std_sigmoid_bwd(int64_t s, int64_t dout) { API_TRY return unary_bwd_impl(k::B_SIGMOID, s, dout); API_CATCH(0) }
int64_t malus_std_relu_bwd(int64_t x, int64_t dout) { API_TRY return unary_bwd_impl(k::B_RELU, x, dout); API_CATCH(0) }
int64_t malus_std_tanh_bwd(int64_t t, int64_t dout) { API_TRY return unary_bwd_impl(k::B_TANH, t, dout); API_CATCH(0) }
int64_t malus_std_sqrt_bwd(int64_t s, int64_t dout) { API_TRY return unary_bwd_impl(k::B_SQRT, s, dout); API_CATCH(0) }
int64_t malus_std_abs_bwd(int64_t x, int64_t dout) { API_TRY return unary_bwd_impl(k::B_ABS, x, dout); API_CATCH(0) }
int64_t malus_std_gelu_bwd(int64_t x, int64_t dout) { API_TRY return unary_bwd_impl(k::B_GELU, x, dout); API_CATCH(0) }

// reduce_bwd.ml:73-76: fill_like(x, dout[0]) with dout[0] read on the device
// (the reference reads it on the host, forcing a flush mid-backward).
int64_t malus_std_sum_bwd(int64_t x, int64_t dout) {
  API_TRY
  TensorBuffer *t = T(x), *d = T(dout);
  TensorBuffer* out = alloc_tensor(F32, t->shape, t->ndim);
  k::fill_from_device(out->f32(), d->f32(), out->len, stream());
  return done(out, "sum_bwd");
  API_CATCH(0)
}

// ---- reduce VJPs (reduce_bwd.ml:40-71) --------------------------------------------
int64_t malus_std_reduce_sum_axis_bwd(int64_t x, int64_t dout, int64_t axis) {
  return malus_std_expand_axis_fwd(dout, x, axis);
}
int64_t malus_std_reduce_mean_axis_bwd(int64_t x, int64_t dout, int64_t axis) {
  API_TRY
  TensorBuffer* t = T(x);
  float n_f = (float)t->shape[norm_axis(axis, t->ndim)];
  int64_t scaled = malus_std_scale_fwd(dout, 1.0f / n_f);
  int64_t r = malus_std_expand_axis_fwd(scaled, x, axis);
  release(T(scaled));
  return r;
  API_CATCH(0)
}
int64_t malus_std_reduce_max_axis_bwd(int64_t x, int64_t y, int64_t dout, int64_t axis) {
  API_TRY
  int64_t y_bc = malus_std_expand_axis_fwd(y, x, axis);
  int64_t mask = malus_std_eq_fwd(x, y_bc);
  int64_t d_bc = malus_std_expand_axis_fwd(dout, x, axis);
  int64_t r = malus_std_broadcast_mul_fwd(d_bc, mask);
  release(T(y_bc)); release(T(mask)); release(T(d_bc));
  return r;
  API_CATCH(0)
}
int64_t malus_std_reduce_var_axis_bwd(int64_t x, int64_t dout, int64_t axis) {
  API_TRY
  TensorBuffer* t = T(x);
  int64_t mean_h = malus_std_reduce_fwd(k::R_MEAN, x, axis, 1);
  int64_t mean_bc = malus_std_expand_axis_fwd(mean_h, x, axis);
  int64_t xm = malus_std_broadcast_sub_fwd(x, mean_bc);
  float n_f = (float)t->shape[norm_axis(axis, t->ndim)];
  int64_t scaled = malus_std_scale_fwd(xm, 2.0f / n_f);
  int64_t d_bc = malus_std_expand_axis_fwd(dout, x, axis);
  int64_t r = malus_std_broadcast_mul_fwd(d_bc, scaled);
  release(T(mean_h)); release(T(mean_bc)); release(T(xm)); release(T(scaled)); release(T(d_bc));
  return r;
  API_CATCH(0)
}

// ---- transformer VJPs (transformer_bwd.ml) -------------------------------------------
int64_t malus_std_softmax_bwd(int64_t s, int64_t dout, int64_t axis) {
  API_TRY
  TensorBuffer *ts = T(s), *td = T(dout);
  if (!same_shape(ts, td)) fail("malus: softmax VJP shape mismatch %s vs %s", shape_str(ts).c_str(), shape_str(td).c_str());
  size_t o, a, in;
  split_axis(ts, norm_axis(axis, ts->ndim), &o, &a, &in);
  TensorBuffer* out = alloc_like(ts);
  k::softmax_bwd(ts->f32(), td->f32(), out->f32(), o, a, in, stream());
  return done(out, "softmax_bwd");
  API_CATCH(0)
}
// tape.rs:1162-1186 (per-row variance broadcast correctly; see layernorm.ml:71)
int64_t malus_std_layernorm_bwd(int64_t y, int64_t var, int64_t dout, int64_t axis) {
  API_TRY
  return layernorm_bwd_impl(y, var, dout, axis, nullptr);
  API_CATCH(0)
}
int64_t malus_std_cross_entropy_bwd(int64_t probs, int64_t targets, int64_t dout) {
  API_TRY
  TensorBuffer *p = T(probs), *tg = T(targets), *d = T(dout);
  bool owned;
  TensorBuffer* ti = as_i32_indices(tg, &owned);
  TensorBuffer* out = alloc_like(p);
  k::ce_bwd(p->f32(), ti->i32(), d->f32(), 0.0f, out->f32(), p->shape[0], p->shape[1], stream());
  return done(out, "cross_entropy_bwd");
  API_CATCH(0)
}
// Fused attention scores: softmax(q @ permute(k, 0, 2, 1) * scale + mask,
// axis=2) for q, k: [bh, t, hs], scale: [1, 1], mask: [t, t].  causal != 0
// promises a causal mask (-1e9 above the diagonal).  Returns 0 with the error
// set for shapes the fused kernel is not built for.
// Checks of the public attention entries.  Every operand is f32.  causal=1
// lets the kernels skip the key tiles above the diagonal, which is only valid
// for the mask tensor_causal_mask builds (0 on and below the diagonal, -1e9
// above; checked here on the host) and, in the VJPs, for probabilities that a
// causal forward wrote (marked on their storage).
static void attn_need_f32(const char* what, std::initializer_list<const TensorBuffer*> ts) {
  for (const TensorBuffer* t : ts)
    if (t && t->dtype != F32) fail("malus: %s: every operand must be f32, got dtype tag %d", what, (int)t->dtype);
}
static void attn_need_causal_mask(const char* what, const TensorBuffer* mk, size_t t) {
  if (!mk->st) fail("malus: %s: the mask has no device storage", what);
  if (mk->st->causal_mask_t == (uint32_t)t && mk->len == t * t) return;  // built by tensor_causal_mask(t)
  std::vector<float> m(t * t);
  download(m.data(), mk, m.size() * sizeof(float));
  for (size_t i = 0; i < t; ++i)
    for (size_t j = 0; j < t; ++j)
      if (m[i * t + j] != (j > i ? -1e9f : 0.0f))
        fail("malus: %s: causal=1 needs the causal mask (0 on/below the diagonal, -1e9 above); element [%zu,%zu] is %g",
             what, i, j, (double)m[i * t + j]);
  mk->st->causal_mask_t = (uint32_t)t;  // verified: later calls skip the download
}
static void attn_need_causal_probs(const char* what, const TensorBuffer* p, size_t t) {
  if (!p->st || p->st->causal_t != (uint32_t)t)
    fail("malus: %s: causal=1 needs probabilities written by a causal attention forward", what);
}

int64_t malus_std_attn_scores_softmax(int64_t q, int64_t kk, int64_t scale, int64_t mask, int32_t causal) {
  API_TRY
  TensorBuffer *Q = T(q), *K = T(kk), *sc = T(scale), *mk = T(mask);
  if (Q->ndim != 3 || K->ndim != 3 || Q->shape[0] != K->shape[0] || Q->shape[1] != K->shape[1] ||
      Q->shape[2] != K->shape[2] || sc->len != 1 || mk->ndim != 2 || mk->shape[0] != Q->shape[1] ||
      mk->shape[1] != Q->shape[1])
    fail("malus: attn_scores_softmax shape mismatch: q %s, k %s, scale %s, mask %s", shape_str(Q).c_str(),
         shape_str(K).c_str(), shape_str(sc).c_str(), shape_str(mk).c_str());
  const size_t bh = Q->shape[0], t = Q->shape[1], hs = Q->shape[2];
  if (!k::attn_scores_supported(bh, t, hs))
    fail("malus: attn_scores_softmax: no fused kernel for t=%zu hs=%zu", t, hs);
  attn_need_f32("attn_scores_softmax", {Q, K, sc, mk});
  if (causal) attn_need_causal_mask("attn_scores_softmax", mk, t);
  const size_t shape[3] = {bh, t, t};
  TensorBuffer* out = alloc_tensor(F32, shape, 3);
  if (!k::attn_scores_softmax(Q->f32(), K->f32(), sc->f32(), mk->f32(), out->f32(), bh, t, hs, causal != 0, stream()))
    fail("malus: attn_scores_softmax: unaligned operand");
  out->st->causal_t = causal ? (uint32_t)t : 0;
  return done(out, "attn_scores_softmax");
  API_CATCH(0)
}
// VJP of the fused scores for dout = d(attn) [bh, t, hs]-shaped heads:
// softmax_bwd(p, dout @ permute(v, 0, 2, 1), axis=2) * scale.
int64_t malus_std_attn_scores_bwd(int64_t dout, int64_t v, int64_t p, int64_t scale, int32_t causal) {
  API_TRY
  TensorBuffer *d = T(dout), *V = T(v), *Pt = T(p), *sc = T(scale);
  if (d->ndim != 3 || V->ndim != 3 || Pt->ndim != 3 || d->shape[0] != V->shape[0] || d->shape[1] != V->shape[1] ||
      d->shape[2] != V->shape[2] || Pt->shape[0] != d->shape[0] || Pt->shape[1] != d->shape[1] ||
      Pt->shape[2] != d->shape[1] || sc->len != 1)
    fail("malus: attn_scores_bwd shape mismatch: dout %s, v %s, p %s, scale %s", shape_str(d).c_str(),
         shape_str(V).c_str(), shape_str(Pt).c_str(), shape_str(sc).c_str());
  const size_t bh = d->shape[0], t = d->shape[1], hs = d->shape[2];
  if (!k::attn_scores_supported(bh, t, hs)) fail("malus: attn_scores_bwd: no fused kernel for t=%zu hs=%zu", t, hs);
  attn_need_f32("attn_scores_bwd", {d, V, Pt, sc});
  if (causal) attn_need_causal_probs("attn_scores_bwd", Pt, t);
  const size_t shape[3] = {bh, t, t};
  TensorBuffer* out = alloc_tensor(F32, shape, 3);
  if (!k::attn_scores_bwd(d->f32(), hs, 1, V->f32(), Pt->f32(), sc->f32(), out->f32(), bh, t, hs, causal != 0, stream()))
    fail("malus: attn_scores_bwd: unaligned operand");
  return done(out, "attn_scores_bwd");
  API_CATCH(0)
}
int64_t malus_std_attn_fwd(int64_t q, int64_t kk, int64_t v, int64_t scale, int64_t mask, int32_t causal,
                           int64_t* p_out) {
  API_TRY
  TensorBuffer *Q = T(q), *K = T(kk), *V = T(v), *sc = T(scale), *mk = T(mask);
  if (Q->ndim != 3 || K->ndim != 3 || V->ndim != 3 || Q->shape[0] != K->shape[0] || Q->shape[1] != K->shape[1] ||
      Q->shape[2] != K->shape[2] || V->shape[0] != Q->shape[0] || V->shape[1] != Q->shape[1] ||
      V->shape[2] != Q->shape[2] || sc->len != 1 || mk->ndim != 2 || mk->shape[0] != Q->shape[1] ||
      mk->shape[1] != Q->shape[1])
    fail("malus: attn_fwd shape mismatch: q %s, k %s, v %s, scale %s, mask %s", shape_str(Q).c_str(),
         shape_str(K).c_str(), shape_str(V).c_str(), shape_str(sc).c_str(), shape_str(mk).c_str());
  const size_t bh = Q->shape[0], t = Q->shape[1], hs = Q->shape[2];
  if (!k::attn_scores_supported(bh, t, hs)) fail("malus: attn_fwd: no fused kernel for t=%zu hs=%zu", t, hs);
  attn_need_f32("attn_fwd", {Q, K, V, sc, mk});
  if (causal) attn_need_causal_mask("attn_fwd", mk, t);
  const size_t pshape[3] = {bh, t, t};
  TensorBuffer* p = alloc_tensor(F32, pshape, 3);
  TensorBuffer* out = alloc_tensor(F32, Q->shape, 3);
  if (!k::attn_fwd(Q->f32(), K->f32(), V->f32(), sc->f32(), mk->f32(), p->f32(), out->f32(), hs, 1, bh, t, hs,
                   causal != 0, stream()))
    fail("malus: attn_fwd: unaligned operand");
  const uint64_t seq = enqueue_mark("attn_fwd");
  p->st->causal_t = causal ? (uint32_t)t : 0;
  p->write_seq = seq;
  out->write_seq = seq;
  if (p_out) *p_out = malus::H(p);
  else release(p);
  return malus::H(out);
  API_CATCH(0)
}
int64_t malus_std_attn_bwd(int64_t dout, int64_t v, int64_t p, int64_t scale, int64_t kk, int32_t causal,
                           int64_t* dq_out) {
  API_TRY
  TensorBuffer *d = T(dout), *V = T(v), *Pt = T(p), *sc = T(scale), *K = T(kk);
  if (d->ndim != 3 || V->ndim != 3 || Pt->ndim != 3 || K->ndim != 3 || d->shape[0] != V->shape[0] ||
      d->shape[1] != V->shape[1] || d->shape[2] != V->shape[2] || Pt->shape[0] != d->shape[0] ||
      Pt->shape[1] != d->shape[1] || Pt->shape[2] != d->shape[1] || sc->len != 1 || K->shape[0] != V->shape[0] ||
      K->shape[1] != V->shape[1] || K->shape[2] != V->shape[2])
    fail("malus: attn_bwd shape mismatch: dout %s, v %s, p %s, scale %s, k %s", shape_str(d).c_str(),
         shape_str(V).c_str(), shape_str(Pt).c_str(), shape_str(sc).c_str(), shape_str(K).c_str());
  const size_t bh = d->shape[0], t = d->shape[1], hs = d->shape[2];
  if (!k::attn_scores_supported(bh, t, hs)) fail("malus: attn_bwd: no fused kernel for t=%zu hs=%zu", t, hs);
  attn_need_f32("attn_bwd", {d, V, Pt, sc, K});
  if (causal) attn_need_causal_probs("attn_bwd", Pt, t);
  const size_t shape[3] = {bh, t, t};
  TensorBuffer* out = alloc_tensor(F32, shape, 3);
  TensorBuffer* dq = dq_out ? alloc_tensor(F32, K->shape, 3) : nullptr;
  if (!k::attn_bwd(d->f32(), hs, 1, V->f32(), Pt->f32(), sc->f32(), out->f32(), K->f32(), dq ? dq->f32() : nullptr,
                   nullptr, bh, t, hs, causal != 0, stream()))
    fail("malus: attn_bwd: unaligned operand");
  const uint64_t seq = enqueue_mark("attn_bwd");
  out->write_seq = seq;
  if (dq) {
    dq->write_seq = seq;
    *dq_out = malus::H(dq);
  }
  return malus::H(out);
  API_CATCH(0)
}
int64_t malus_std_attn_bwd_all(int64_t dout, int64_t q, int64_t kk, int64_t v, int64_t p, int64_t scale, int32_t causal,
                               int64_t dq_add, int64_t dk_add, int64_t dv_add, int64_t* dq_out, int64_t* dk_out,
                               int64_t* dv_out) {
  API_TRY
  TensorBuffer *d = T(dout), *Q = T(q), *K = T(kk), *V = T(v), *Pt = T(p), *sc = T(scale);
  TensorBuffer *Aq = dq_add ? T(dq_add) : nullptr, *Ak = dk_add ? T(dk_add) : nullptr, *Av = dv_add ? T(dv_add) : nullptr;
  auto same3 = [&](const TensorBuffer* x) {
    return x->ndim == 3 && x->shape[0] == d->shape[0] && x->shape[1] == d->shape[1] && x->shape[2] == d->shape[2];
  };
  if (d->ndim != 3 || !same3(Q) || !same3(K) || !same3(V) || Pt->ndim != 3 || Pt->shape[0] != d->shape[0] ||
      Pt->shape[1] != d->shape[1] || Pt->shape[2] != d->shape[1] || sc->len != 1 || !dq_out || !dk_out || !dv_out ||
      (Aq && !same3(Aq)) || (Ak && !same3(Ak)) || (Av && !same3(Av)))
    fail("malus: attn_bwd_all shape mismatch: dout %s, q %s, k %s, v %s, p %s, scale %s", shape_str(d).c_str(),
         shape_str(Q).c_str(), shape_str(K).c_str(), shape_str(V).c_str(), shape_str(Pt).c_str(),
         shape_str(sc).c_str());
  const size_t bh = d->shape[0], t = d->shape[1], hs = d->shape[2];
  if (!k::attn_scores_supported(bh, t, hs)) fail("malus: attn_bwd_all: no fused kernel for t=%zu hs=%zu", t, hs);
  attn_need_f32("attn_bwd_all", {d, Q, K, V, Pt, sc, Aq, Ak, Av});
  if (causal) attn_need_causal_probs("attn_bwd_all", Pt, t);
  const size_t shape[3] = {bh, t, t};
  TensorBuffer* out = alloc_tensor(F32, shape, 3);
  TensorBuffer *dq = alloc_like(Q), *dk = alloc_like(K), *dv = alloc_like(V);
  const k::AttnKV kv{Q->f32(), dk->f32(), Ak ? Ak->f32() : nullptr, dv->f32(), Av ? Av->f32() : nullptr};
  if (!k::attn_bwd(d->f32(), hs, 1, V->f32(), Pt->f32(), sc->f32(), out->f32(), K->f32(), dq->f32(),
                   Aq ? Aq->f32() : nullptr, bh, t, hs, causal != 0, stream(), &kv))
    fail("malus: attn_bwd_all: unaligned operand");
  const uint64_t seq = enqueue_mark("attn_bwd_all");
  for (TensorBuffer* x : {out, dq, dk, dv}) x->write_seq = seq;
  *dq_out = malus::H(dq);
  *dk_out = malus::H(dk);
  *dv_out = malus::H(dv);
  return malus::H(out);
  API_CATCH(0)
}
// Flash attention (k_flash.hip): q, k, v and the output dense [bh, t, hs],
// lse [bh, t]; causal 0 means no mask.
int64_t malus_std_flash_attn_fwd(int64_t q, int64_t kk, int64_t v, int64_t scale, int32_t causal, int64_t* lse_out) {
  API_TRY
  TensorBuffer *Q = T(q), *K = T(kk), *V = T(v), *sc = T(scale);
  auto same3 = [&](const TensorBuffer* x) {
    return x->ndim == 3 && x->shape[0] == Q->shape[0] && x->shape[1] == Q->shape[1] && x->shape[2] == Q->shape[2];
  };
  if (Q->ndim != 3 || !same3(K) || !same3(V) || sc->len != 1)
    fail("malus: flash_attn_fwd shape mismatch: q %s, k %s, v %s, scale %s", shape_str(Q).c_str(),
         shape_str(K).c_str(), shape_str(V).c_str(), shape_str(sc).c_str());
  const size_t bh = Q->shape[0], t = Q->shape[1], hs = Q->shape[2];
  if (!k::flash_supported(bh, t, hs))
    fail("malus: flash_attn_fwd: t=%zu hs=%zu (needs t a multiple of 32 and hs 32 or 64)", t, hs);
  attn_need_f32("flash_attn_fwd", {Q, K, V, sc});
  const size_t lsh[2] = {bh, t};
  TensorBuffer* lse = alloc_tensor(F32, lsh, 2);
  TensorBuffer* out = alloc_tensor(F32, Q->shape, 3);
  if (!k::flash_fwd(Q->f32(), K->f32(), V->f32(), sc->f32(), out->f32(), hs, 1, lse->f32(), bh, t, hs, causal != 0,
                    k::autocast_on(), stream()))
    fail("malus: flash_attn_fwd: unaligned operand");
  const uint64_t seq = enqueue_mark("flash_attn_fwd");
  out->write_seq = seq;
  lse->write_seq = seq;
  if (lse_out) *lse_out = malus::H(lse);
  else release(lse);
  return malus::H(out);
  API_CATCH(0)
}
int32_t malus_std_flash_attn_bwd(int64_t dout, int64_t q, int64_t kk, int64_t v, int64_t out, int64_t lse,
                                 int64_t scale, int32_t causal, int64_t dq_add, int64_t dk_add, int64_t dv_add,
                                 int64_t* dq_out, int64_t* dk_out, int64_t* dv_out) {
  API_TRY
  TensorBuffer *d = T(dout), *Q = T(q), *K = T(kk), *V = T(v), *O = T(out), *L = T(lse), *sc = T(scale);
  TensorBuffer *Aq = dq_add ? T(dq_add) : nullptr, *Ak = dk_add ? T(dk_add) : nullptr, *Av = dv_add ? T(dv_add) : nullptr;
  auto same3 = [&](const TensorBuffer* x) {
    return x->ndim == 3 && x->shape[0] == d->shape[0] && x->shape[1] == d->shape[1] && x->shape[2] == d->shape[2];
  };
  if (d->ndim != 3 || !same3(Q) || !same3(K) || !same3(V) || !same3(O) || L->len != d->shape[0] * d->shape[1] ||
      sc->len != 1 || !dq_out || !dk_out || !dv_out || (Aq && !same3(Aq)) || (Ak && !same3(Ak)) || (Av && !same3(Av)))
    fail("malus: flash_attn_bwd shape mismatch: dout %s, q %s, k %s, v %s, out %s, lse %s", shape_str(d).c_str(),
         shape_str(Q).c_str(), shape_str(K).c_str(), shape_str(V).c_str(), shape_str(O).c_str(), shape_str(L).c_str());
  const size_t bh = d->shape[0], t = d->shape[1], hs = d->shape[2];
  if (!k::flash_supported(bh, t, hs))
    fail("malus: flash_attn_bwd: t=%zu hs=%zu (needs t a multiple of 32 and hs 32 or 64)", t, hs);
  attn_need_f32("flash_attn_bwd", {d, Q, K, V, O, L, sc, Aq, Ak, Av});
  TensorBuffer *dq = alloc_like(Q), *dk = alloc_like(K), *dv = alloc_like(V);
  size_t bucket;
  float* dsum = static_cast<float*>(pool_alloc(bh * t * sizeof(float), &bucket));
  const k::FlashBwd a{Q->f32(), K->f32(), V->f32(), O->f32(), d->f32(), L->f32(), sc->f32(),
                      dq->f32(), dk->f32(), dv->f32(), dsum,
                      Aq ? Aq->f32() : nullptr, Ak ? Ak->f32() : nullptr, Av ? Av->f32() : nullptr};
  if (!k::flash_bwd(a, hs, 1, bh, t, hs, causal != 0, k::autocast_on(), stream()))
    fail("malus: flash_attn_bwd: unaligned operand");
  pool_free(dsum, bucket);  // stream order: later users of the buffer run after the kernels
  const uint64_t seq = enqueue_mark("flash_attn_bwd");
  for (TensorBuffer* x : {dq, dk, dv}) x->write_seq = seq;
  *dq_out = malus::H(dq);
  *dk_out = malus::H(dk);
  *dv_out = malus::H(dv);
  return 0;
  API_CATCH(-1)
}
int64_t malus_std_embedding_bwd(int64_t weight, int64_t indices, int64_t dout) {
  API_TRY
  TensorBuffer *w = T(weight), *idx = T(indices), *d = T(dout);
  bool owned;
  TensorBuffer* ii = as_i32_indices(idx, &owned);
  TensorBuffer* out = alloc_tensor(F32, w->shape, 2);
  k::embedding_bwd(d->f32(), ii->i32(), out->f32(), idx->len, w->shape[0], w->shape[1], stream());
  return done(out, "embedding_bwd");
  API_CATCH(0)
}

}  // extern "C"

bool embedding_bwd2_impl(int64_t wa, int64_t ia, int64_t wb, int64_t ib, int64_t dout, int64_t* dwa, int64_t* dwb) {
  TensorBuffer *A = T(wa), *IA = T(ia), *B = T(wb), *IB = T(ib), *d = T(dout);
  if (A->ndim != 2 || B->ndim != 2 || A->shape[1] != B->shape[1] || IA->dtype != I32 || IB->dtype != I32 ||
      IA->len != IB->len || d->dtype != F32 || d->len != IA->len * A->shape[1])
    return false;
  TensorBuffer* oa = alloc_tensor(F32, A->shape, 2);
  TensorBuffer* ob = alloc_tensor(F32, B->shape, 2);
  if (!k::embedding_bwd2(d->f32(), IA->i32(), oa->f32(), A->shape[0], IB->i32(), ob->f32(), B->shape[0], IA->len,
                         A->shape[1], stream())) {
    release(oa);
    release(ob);
    return false;
  }
  const uint64_t seq = enqueue_mark("embedding_bwd2");
  oa->write_seq = ob->write_seq = seq;
  *dwa = malus::H(oa);
  *dwb = malus::H(ob);
  return true;
}

// ---- matmul (metal.rs:820-962) and its VJPs (matmul_bwd.ml:15-29) ---------------------
// The *_impl forms take an optional addend D of the output's shape and
// return D + product (one GEMM, the product rounded before the add), which
// is how a gradient accumulation or residual add folds into the GEMM.
int64_t matmul_impl(int64_t ha, int64_t hb, const TensorBuffer* D) {
  TensorBuffer *a = T(ha), *b = T(hb);
  gemm_io(a, b, "matmul");
  if (a->ndim == 2 && b->ndim == 2) {
    size_t m = a->shape[0], k = a->shape[1], k2 = b->shape[0], n = b->shape[1];
    if (k != k2)
      fail("malus: matmul shape mismatch: [%zux%zu] @ [%zux%zu] - inner dims %zu != %zu\n  left shape:  %s\n  right shape: %s",
           m, k, k2, n, k, k2, shape_str(a).c_str(), shape_str(b).c_str());
    size_t osh[2] = {m, n};
    return gemm_out(a, b, false, false, 1, (int)m, (int)n, (int)k, 0, 0, osh, 2, D);
  }
  if (a->ndim == 3 && b->ndim == 3) {
    size_t bt = a->shape[0], m = a->shape[1], k = a->shape[2], bt2 = b->shape[0], k2 = b->shape[1], n = b->shape[2];
    if (bt != bt2)
      fail("malus: batched matmul batch dims must match: %zu vs %zu\n  left shape:  %s\n  right shape: %s", bt, bt2,
           shape_str(a).c_str(), shape_str(b).c_str());
    if (k != k2)
      fail("malus: batched matmul inner dims must match: %zu vs %zu\n  left shape:  %s\n  right shape: %s", k, k2,
           shape_str(a).c_str(), shape_str(b).c_str());
    size_t osh[3] = {bt, m, n};
    return gemm_out(a, b, false, false, (int)bt, (int)m, (int)n, (int)k, (long)(m * k), (long)(k * n), osh, 3, D);
  }
  if (a->ndim == 3 && b->ndim == 2) {  // weight broadcast over the batch: one [B*M, K] GEMM
    size_t bt = a->shape[0], m = a->shape[1], k = a->shape[2], k2 = b->shape[0], n = b->shape[1];
    if (k != k2)
      fail("malus: matmul shape mismatch: [%zux%zux%zu] @ [%zux%zu] - inner dims %zu != %zu\n  left shape:  %s\n  right shape: %s",
           bt, m, k, k2, n, k, k2, shape_str(a).c_str(), shape_str(b).c_str());
    size_t osh[3] = {bt, m, n};
    return gemm_out(a, b, false, false, 1, (int)(bt * m), (int)n, (int)k, 0, 0, osh, 3, D);
  }
  fail("malus: tensor_matmul requires both inputs to be 2-D, both 3-D, or (3-D, 2-D)\n  left shape:  %s\n  right shape: %s",
       shape_str(a).c_str(), shape_str(b).c_str());
}

// transformer_bwd.ml:24-36 with the per-row variance (tape.rs:1162-1186);
// with D, returns D + dx (gradient accumulation folded into the kernel).
int64_t layernorm_bwd_impl(int64_t y, int64_t var, int64_t dout, int64_t axis, const TensorBuffer* D) {
  TensorBuffer *ty = T(y), *tv = T(var), *td = T(dout);
  int ax = norm_axis(axis, ty->ndim);
  size_t o, a, in;
  split_axis(ty, ax, &o, &a, &in);
  if (tv->len != o * in) fail("malus: layernorm VJP expects a keepdim variance of %zu elements, got %zu", o * in, tv->len);
  if (D && (D->dtype != F32 || D->len != ty->len))
    fail("malus: layernorm VJP accumulate: addend %s does not match %s", shape_str(D).c_str(), shape_str(ty).c_str());
  TensorBuffer* out = alloc_like(ty);
  k::layernorm_bwd(ty->f32(), tv->f32(), td->f32(), out->f32(), o, a, in, 1e-5f, stream(), D ? D->f32() : nullptr);
  return done(out, "layernorm_bwd");
}

// out = layernorm(x, axis=-1) * w (nanogpt_modular.ml:47 and :62) from one
// kernel; *y_out gets the normalized rows, *var_out the keepdim variance.
// out_bf16: out is stored in bf16 (rounded to nearest even), for a caller
// whose only readers of it are bf16 GEMMs.
int64_t ln_affine_fwd(int64_t hx, int64_t hw, int64_t* y_out, int64_t* var_out, bool out_bf16) {
  TensorBuffer *t = T(hx), *w = T(hw);
  need_f32(t, "layernorm");
  const size_t a = t->shape[t->ndim - 1];
  if (w->len != a || w->dtype != F32)
    fail("malus: fused layernorm scale: weight %s does not match the last axis of %s", shape_str(w).c_str(),
         shape_str(t).c_str());
  TensorBuffer* y = alloc_like(t);
  TensorBuffer* out = alloc_tensor(out_bf16 ? BF16 : F32, t->shape, t->ndim);
  size_t vsh[kMaxRank];
  for (int i = 0; i < t->ndim; ++i) vsh[i] = i == t->ndim - 1 ? 1 : t->shape[i];
  TensorBuffer* var = alloc_tensor(F32, vsh, t->ndim);
  k::layernorm(t->f32(), y->f32(), var->f32(), t->len / a, a, 1, 1e-5f, stream(), w->f32(), out->f32(), out_bf16);
  uint64_t seq = enqueue_mark("layernorm_affine");
  y->write_seq = var->write_seq = out->write_seq = seq;
  *y_out = H(y);
  *var_out = H(var);
  return H(out);
}
// dx of out = layernorm(x) * w: the layernorm VJP of dout * w (+ D)
int64_t ln_affine_bwd_x(int64_t hy, int64_t hvar, int64_t hw, int64_t hd, const TensorBuffer* D) {
  TensorBuffer *ty = T(hy), *tv = T(hvar), *tw = T(hw), *td = T(hd);
  const size_t a = ty->shape[ty->ndim - 1], o = ty->len / a;
  if (tv->len != o || tw->len != a || td->len != ty->len)
    fail("malus: fused layernorm scale VJP: y %s, var %s, w %s, dout %s", shape_str(ty).c_str(), shape_str(tv).c_str(),
         shape_str(tw).c_str(), shape_str(td).c_str());
  if (D && (D->dtype != F32 || D->len != ty->len))
    fail("malus: layernorm VJP accumulate: addend %s does not match %s", shape_str(D).c_str(), shape_str(ty).c_str());
  TensorBuffer* out = alloc_like(ty);
  k::layernorm_bwd(ty->f32(), tv->f32(), td->f32(), out->f32(), o, a, 1, 1e-5f, stream(), D ? D->f32() : nullptr,
                   tw->f32());
  return done(out, "layernorm_affine_bwd");
}

// ln_affine_bwd_x and the scale's gradient mul_bwd_b(dout, y, w) from one
// row kernel (bit-identical to the two calls); *dw_out gets dw.  0 when the
// shape has no fused form (nothing launched).
int64_t ln_affine_bwd_xw(int64_t hy, int64_t hvar, int64_t hw, int64_t hd, const TensorBuffer* D, int64_t* dw_out,
                         bool defer_dw) {
  TensorBuffer *ty = T(hy), *tv = T(hvar), *tw = T(hw), *td = T(hd);
  const size_t a = ty->shape[ty->ndim - 1], o = ty->len / a;
  if (tv->len != o || tw->len != a || td->len != ty->len || tw->ndim != 1) return 0;
  if (D && (D->dtype != F32 || D->len != ty->len))
    fail("malus: layernorm VJP accumulate: addend %s does not match %s", shape_str(D).c_str(), shape_str(ty).c_str());
  TensorBuffer* out = alloc_like(ty);
  TensorBuffer* dw = alloc_tensor(F32, tw->shape, tw->ndim);
  if (!k::layernorm_bwd_scale(ty->f32(), tv->f32(), td->f32(), out->f32(), dw->f32(), o, a, 1e-5f, stream(),
                              D ? D->f32() : nullptr, tw->f32(), defer_dw)) {
    release(out);
    release(dw);
    return 0;
  }
  const uint64_t seq = enqueue_mark("layernorm_affine_bwd_xw");
  out->write_seq = seq;
  dw->write_seq = seq;
  *dw_out = malus::H(dw);
  return malus::H(out);
}

// h = x @ W1 and ge = gelu(h) from one GEMM (nanogpt_modular.ml:63);
// returns h, *ge_out gets gelu(h).  0 when the shape does not fit the fused
// epilogue (nothing launched).  x may be bf16; ge_bf16 stores ge in bf16
// (for a caller whose readers of ge are bf16 GEMMs); h stays f32.
int64_t matmul_gelu_fwd(int64_t hx, int64_t hw, int64_t* ge_out, bool ge_bf16) {
  const TensorBuffer *x = gemm_operand(T(hx)), *w = gemm_operand(T(hw), true);
  if (x->ndim != 2 || w->ndim != 2 || x->shape[1] != w->shape[0]) return 0;
  const int io = gemm_io(x, w, "matmul") | (ge_bf16 ? k::kIoE16 : 0);
  const size_t M = x->shape[0], K = x->shape[1], N = w->shape[1];
  const size_t sh[2] = {M, N};
  TensorBuffer* h = alloc_tensor(F32, sh, 2);
  TensorBuffer* ge = alloc_tensor(ge_bf16 ? BF16 : F32, sh, 2);
  KTimer* kt = ktimer_begin("gemm");
  if (!k::gemm_gelu(x->f32(), w->f32(), h->f32(), ge->f32(), (int)M, (int)N, (int)K, false, false, stream(), nullptr,
                    io)) {
    ktimer_end(kt, 0);
    release(h);
    release(ge);
    return 0;
  }
  ktimer_end(kt, 2.0 * M * N * K);
  h->write_seq = ge->write_seq = enqueue_mark("matmul_gelu");
  *ge_out = H(ge);
  return H(h);
}
// dh of mo = gelu(h) @ W2: gelu_bwd(h, dout @ W2^T) (+ D) from one GEMM;
// out_bf16 stores dh in bf16 (no D) for a caller whose readers of dh are
// bf16 GEMMs.
int64_t gelu_matmul_bwd_h(int64_t hd, int64_t hw, int64_t hh, const TensorBuffer* D, bool out_bf16) {
  const TensorBuffer *d = T(hd), *w = gemm_operand(T(hw)), *h = T(hh);
  const size_t N = w->shape[0], K = w->shape[1], M = d->len / K;
  if (h->len != M * N || d->len != M * K) fail("malus: gelu matmul VJP: dout %s, w %s, h %s", shape_str(d).c_str(),
                                               shape_str(w).c_str(), shape_str(h).c_str());
  if (D && (D->dtype != F32 || D->len != h->len))
    fail("malus: gelu matmul VJP accumulate: addend %s does not match %s", shape_str(D).c_str(), shape_str(h).c_str());
  need_f32(d, "gelu matmul VJP");
  need_f32(h, "gelu matmul VJP");
  const int io = gemm_io(d, w, "gelu matmul VJP") | (out_bf16 ? k::kIoC16 : 0);
  if (D && out_bf16) fail("malus: gelu matmul VJP: a bf16 result takes no addend");
  TensorBuffer* out = alloc_tensor(out_bf16 ? BF16 : F32, h->shape, h->ndim);
  KTimer* kt = ktimer_begin("gemm");
  if (!k::gemm_gelu(d->f32(), w->f32(), out->f32(), h->f32(), (int)M, (int)N, (int)K, true, true, stream(),
                    D ? D->f32() : nullptr, io))
    fail("malus: gelu matmul VJP: no fused GEMM for %zux%zux%zu", M, N, K);
  ktimer_end(kt, 2.0 * M * N * K);
  return done(out, "gelu_matmul_bwd");
}

// dA = dout @ op(B)^T
int64_t matmul_bwd_a_impl(int64_t ha, int64_t hb, int64_t hd, const TensorBuffer* D) {
  TensorBuffer *a = T(ha), *b = T(hb), *d = T(hd);
  if (b->ndim == 3) {  // 3x3: dout[b] @ B[b]^T
    size_t bt = d->shape[0], m = d->shape[1], n = d->shape[2], k = b->shape[1];
    return gemm_out(d, b, false, true, (int)bt, (int)m, (int)k, (int)n, (long)(m * n), (long)(k * n), a->shape, a->ndim, D);
  }
  // b is 2-D [K, N]; dout is [.., N] flattened to rows
  size_t n = b->shape[1], k = b->shape[0], rows = d->len / n;
  return gemm_out(d, b, false, true, 1, (int)rows, (int)k, (int)n, 0, 0, a->shape, a->ndim, D);
}

// dB = op(A)^T @ dout (the 3x2 case sums over the batch inside one GEMM)
int64_t matmul_bwd_b_impl(int64_t ha, int64_t hb, int64_t hd, const TensorBuffer* D) {
  TensorBuffer *a = T(ha), *b = T(hb), *d = T(hd);
  if (a->ndim == 3 && b->ndim == 3) {
    size_t bt = a->shape[0], m = a->shape[1], k = a->shape[2], n = d->shape[2];
    return gemm_out(a, d, true, false, (int)bt, (int)k, (int)n, (int)m, (long)(m * k), (long)(m * n), b->shape, b->ndim, D);
  }
  // A flattened to [rows, K] (2-D, or 3-D with B broadcast): A^T @ dout[rows, N]
  size_t k = a->shape[a->ndim - 1], rows = a->len / k, n = d->shape[d->ndim - 1];
  return gemm_out(a, d, true, false, 1, (int)k, (int)n, (int)rows, 0, 0, b->shape, b->ndim, D);
}

// ---- head-folded attention GEMMs (nanogpt_modular.ml:49-60) -----------------
// The composed attention moves each [B*T, C] projection into heads with
// reshape(permute(reshape(x @ W, B, T, H, hs), 0, 2, 1, 3), B*H, T, hs) and
// back with the inverse chain; permute is an exact copy, so these GEMMs read
// and write the folded layouts in place instead.  Values, and the order of
// every sum, are those of the composed ops.
using k::dense_layout;
using k::GemmLayout;
using k::GemmLayouts;
namespace {
TensorBuffer* T_(int64_t h) { return malus::T(h); }  // T is a sequence length below
// [B*T, C] matrix stored as [B, H, T, hs] (row m = b T + t, column n = h hs + d)
GemmLayout heads_as_rows(int T, int H, int hs) {
  return {{0, 0, 0}, {T, T * H * hs, hs}, {hs, T * hs, 1}};
}
// per-head [T, hs] matrices of batch bh = b H + h stored inside [B, T, H, hs]
GemmLayout rows_as_heads(int T, int H, int hs) {
  return {{H, T * H * hs, hs}, {0, 0, H * hs}, {0, 0, 1}};
}
void check_addend(const TensorBuffer* D, const TensorBuffer* c) {
  if (D && (D->dtype != F32 || D->len != c->len))
    fail("malus: fused attention accumulate: addend %s does not match %s", shape_str(D).c_str(), shape_str(c).c_str());
}
int64_t mapped(const TensorBuffer* a, const TensorBuffer* b, TensorBuffer* c, bool ta, bool tb, int batch, int M, int N,
               int K, const GemmLayouts& L, const TensorBuffer* D, const char* what) {
  check_addend(D, c);
  a = gemm_operand(a);
  b = gemm_operand(b, !ta && !tb);
  GemmLayouts Lio = L;
  Lio.io = gemm_io(a, b, what);
  KTimer* kt = ktimer_begin("gemm");
  double flops = 0;
  if (!k::gemm_mapped(a->f32(), b->f32(), c->f32(), batch, M, N, K, ta, tb, Lio, stream(), D ? D->f32() : nullptr,
                      &flops))
    fail("malus: %s: head-folded GEMM layout rejected (T %% 32, hs %% 16 and sizes below 2 GiB are required)", what);
  ktimer_end(kt, flops);  // executed work: causal GEMMs skip the zero triangle
  return done(c, what);
}
}  // namespace

bool heads_foldable(size_t B, size_t T, size_t H, size_t hs) {
  const size_t n = B * T * H * hs;
  return T % 32 == 0 && hs % 16 == 0 && B * H <= 65535 && n * 4 < (1ull << 31) && T * T * B * H * 4 < (1ull << 31);
}

// Qh = heads(x @ W): x [B*T, C], W [C, C] -> [B*H, T, hs]
int64_t head_proj_fwd(int64_t hx, int64_t hw, size_t B, size_t T, size_t H) {
  TensorBuffer *x = T_(hx), *w = T_(hw);
  const size_t C = w->shape[1], hs = C / H, N = B * T;
  const size_t sh[3] = {B * H, T, hs};
  TensorBuffer* c = alloc_tensor(F32, sh, 3);
  GemmLayouts L{dense_layout((long)x->shape[1], 0), dense_layout((long)C, 0), heads_as_rows(T, H, hs),
                (int)x->len, (int)w->len};
  return mapped(x, w, c, false, false, 1, (int)N, (int)C, (int)w->shape[0], L, nullptr, "head_proj");
}
// dx = unheads(dQh) @ W^T  (+ D)
int64_t head_proj_bwd_x(int64_t hdq, int64_t hw, size_t B, size_t T, size_t H, const TensorBuffer* D) {
  TensorBuffer *dq = T_(hdq), *w = T_(hw);
  const size_t Cin = w->shape[0], C = w->shape[1], hs = C / H, N = B * T;
  const size_t sh[2] = {N, Cin};
  TensorBuffer* c = alloc_tensor(F32, sh, 2);
  GemmLayouts L{heads_as_rows(T, H, hs), dense_layout((long)C, 0), dense_layout((long)Cin, 0), (int)dq->len,
                (int)w->len};
  return mapped(dq, w, c, false, true, 1, (int)N, (int)Cin, (int)C, L, D, "head_proj_bwd_x");
}
// dW = x^T @ unheads(dQh)  (+ D)
int64_t head_proj_bwd_w(int64_t hx, int64_t hdq, size_t B, size_t T, size_t H, const TensorBuffer* D) {
  TensorBuffer *x = T_(hx), *dq = T_(hdq);
  const size_t Cin = x->shape[1], hs = dq->shape[2], C = H * hs, N = B * T;
  const size_t sh[2] = {Cin, C};
  TensorBuffer* c = alloc_tensor(F32, sh, 2);
  GemmLayouts L{dense_layout((long)Cin, 0), heads_as_rows(T, H, hs), dense_layout((long)C, 0), (int)x->len,
                (int)dq->len};
  return mapped(x, dq, c, true, false, 1, (int)Cin, (int)C, (int)N, L, D, "head_proj_bwd_w");
}
// Qh_g = heads(x @ W_g) for three weights in one launch.
void head_proj_fwd3(int64_t hx, const int64_t* hw, size_t B, size_t T, size_t H, int64_t* out, bool out_bf16) {
  TensorBuffer* x = T_(hx);
  TensorBuffer* w0 = T_(hw[0]);
  const size_t C = w0->shape[1], hs = C / H, N = B * T;
  const size_t sh[3] = {B * H, T, hs};
  GemmLayouts L{dense_layout((long)x->shape[1], 0), dense_layout((long)C, 0), heads_as_rows(T, H, hs), (int)x->len,
                (int)w0->len};
  L.ngroup = 3;
  const TensorBuffer* w[3] = {gemm_operand(w0, true), gemm_operand(T_(hw[1]), true), gemm_operand(T_(hw[2]), true)};
  L.io = gemm_io(x, w[0], "head_proj_fwd3") | (out_bf16 ? k::kIoC16 : 0);
  TensorBuffer* o[3];
  for (int g = 0; g < 3; ++g) {
    if (w[g]->len != w0->len || w[g]->dtype != w[0]->dtype) fail("malus: head_proj_fwd3: weights differ in shape or dtype");
    o[g] = alloc_tensor(out_bf16 ? BF16 : F32, sh, 3);
    L.ga[g] = x->f32();
    L.gb[g] = w[g]->f32();
    L.gc[g] = o[g]->f32();
  }
  KTimer* kt = ktimer_begin("gemm");
  double flops = 0;
  if (!k::gemm_grouped((int)N, (int)C, (int)w0->shape[0], false, false, L, nullptr, false, stream(), nullptr, &flops))
    fail("malus: head_proj_fwd3: grouped GEMM rejected");
  ktimer_end(kt, flops);
  const uint64_t seq = enqueue_mark("head_proj3");
  for (int g = 0; g < 3; ++g) {
    o[g]->write_seq = seq;
    out[g] = malus::H(o[g]);
  }
}

// The three projections of one input (q, k, v) in one launch each:
// dx = ((D + unheads(dQh_0) @ W_0^T) + unheads(dQh_1) @ W_1^T) + unheads(dQh_2) @ W_2^T,
// in the given group order (the tape's order), and dW_g = x^T @ unheads(dQh_g).
int64_t head_proj_bwd_x3(const int64_t* hdq, const int64_t* hw, size_t B, size_t T, size_t H, const TensorBuffer* D) {
  TensorBuffer* w0 = T_(hw[0]);
  const size_t Cin = w0->shape[0], C = w0->shape[1], hs = C / H, N = B * T;
  const size_t sh[2] = {N, Cin};
  TensorBuffer* c = alloc_tensor(F32, sh, 2);
  check_addend(D, c);
  GemmLayouts L{heads_as_rows(T, H, hs), dense_layout((long)C, 0), dense_layout((long)Cin, 0), (int)T_(hdq[0])->len,
                (int)w0->len};
  L.ngroup = 3;
  const TensorBuffer* w[3] = {gemm_operand(w0), gemm_operand(T_(hw[1])), gemm_operand(T_(hw[2]))};
  L.io = gemm_io(T_(hdq[0]), w[0], "head_proj_bwd_x3");
  for (int g = 0; g < 3; ++g) {
    if (T_(hdq[g])->dtype != T_(hdq[0])->dtype || w[g]->dtype != w[0]->dtype)
      fail("malus: head_proj_bwd_x3: gradients or weights differ in dtype");
    L.ga[g] = T_(hdq[g])->f32();
    L.gb[g] = w[g]->f32();
  }
  KTimer* kt = ktimer_begin("gemm");
  double flops = 0;
  if (!k::gemm_grouped((int)N, (int)Cin, (int)C, false, true, L, c->f32(), true, stream(), D ? D->f32() : nullptr,
                       &flops))
    fail("malus: head_proj_bwd_x3: grouped GEMM rejected");
  ktimer_end(kt, flops);
  return done(c, "head_proj_bwd_x3");
}
void head_proj_bwd_w3(int64_t hx, const int64_t* hdq, size_t B, size_t T, size_t H, int64_t* out) {
  TensorBuffer* x = T_(hx);
  const size_t Cin = x->shape[1], hs = T_(hdq[0])->shape[2], C = H * hs, N = B * T;
  const size_t sh[2] = {Cin, C};
  GemmLayouts L{dense_layout((long)Cin, 0), heads_as_rows(T, H, hs), dense_layout((long)C, 0), (int)x->len,
                (int)T_(hdq[0])->len};
  L.ngroup = 3;
  L.io = gemm_io(x, T_(hdq[0]), "head_proj_bwd_w3");
  TensorBuffer* o[3];
  for (int g = 0; g < 3; ++g) {
    if (T_(hdq[g])->dtype != T_(hdq[0])->dtype) fail("malus: head_proj_bwd_w3: gradients differ in dtype");
    o[g] = alloc_tensor(F32, sh, 2);
    L.ga[g] = x->f32();
    L.gb[g] = T_(hdq[g])->f32();
    L.gc[g] = o[g]->f32();
  }
  KTimer* kt = ktimer_begin("gemm");
  double flops = 0;
  if (!k::gemm_grouped((int)Cin, (int)C, (int)N, true, false, L, nullptr, false, stream(), nullptr, &flops))
    fail("malus: head_proj_bwd_w3: grouped GEMM rejected");
  ktimer_end(kt, flops);
  const uint64_t seq = enqueue_mark("head_proj_bwd_w3");
  for (int g = 0; g < 3; ++g) {
    o[g]->write_seq = seq;
    out[g] = malus::H(o[g]);
  }
}

// att = unheads(P @ V): P [B*H, T, T], V [B*H, T, hs] -> [B*T, H*hs]
int64_t attn_out_fwd(int64_t hp, int64_t hv, size_t B, size_t T, size_t H, bool causal) {
  TensorBuffer *p = T_(hp), *v = T_(hv);
  const size_t hs = v->shape[2], C = H * hs, N = B * T;
  const size_t sh[2] = {N, C};
  TensorBuffer* c = alloc_tensor(F32, sh, 2);
  GemmLayouts L{dense_layout((long)T, (long)(T * T)), dense_layout((long)hs, (long)(T * hs)), rows_as_heads(T, H, hs),
                (int)p->len, (int)v->len, causal ? 1 : 0};
  return mapped(p, v, c, false, false, (int)(B * H), (int)T, (int)hs, (int)T, L, nullptr, "attn_out");
}
// dP = heads(dAtt) @ V^T  (+ D)
int64_t attn_out_bwd_p(int64_t hda, int64_t hv, size_t B, size_t T, size_t H, const TensorBuffer* D) {
  TensorBuffer *da = T_(hda), *v = T_(hv);
  const size_t hs = v->shape[2];
  const size_t sh[3] = {B * H, T, T};
  TensorBuffer* c = alloc_tensor(F32, sh, 3);
  GemmLayouts L{rows_as_heads(T, H, hs), dense_layout((long)hs, (long)(T * hs)), dense_layout((long)T, (long)(T * T)),
                (int)da->len, (int)v->len};
  return mapped(da, v, c, false, true, (int)(B * H), (int)T, (int)T, (int)hs, L, D, "attn_out_bwd_p");
}
// dV = P^T @ heads(dAtt)  (+ D)
int64_t attn_out_bwd_v(int64_t hp, int64_t hda, size_t B, size_t T, size_t H, const TensorBuffer* D, bool causal) {
  TensorBuffer *p = T_(hp), *da = T_(hda);
  const size_t hs = da->shape[1] / H;
  const size_t sh[3] = {B * H, T, hs};
  TensorBuffer* c = alloc_tensor(F32, sh, 3);
  GemmLayouts L{dense_layout((long)T, (long)(T * T)), rows_as_heads(T, H, hs), dense_layout((long)hs, (long)(T * hs)),
                (int)p->len, (int)da->len, causal ? 1 : 0};
  return mapped(p, da, c, true, false, (int)(B * H), (int)T, (int)hs, (int)T, L, D, "attn_out_bwd_v");
}
// dS of the fused causal attention: softmax_bwd(P, heads(dAtt) @ V^T) * scale
int64_t attn_scores_bwd_impl(int64_t hda, int64_t hv, int64_t hp, int64_t hscale, size_t B, size_t T, size_t H) {
  TensorBuffer *da = T_(hda), *v = T_(hv), *p = T_(hp), *sc = T_(hscale);
  const size_t hs = v->shape[2], bh = B * H;
  const size_t sh[3] = {bh, T, T};
  TensorBuffer* out = alloc_tensor(F32, sh, 3);
  if (!k::attn_scores_bwd(da->f32(), H * hs, H, v->f32(), p->f32(), sc->f32(), out->f32(), bh, T, hs, true, stream()))
    fail("malus: attn_scores_bwd: no fused kernel for t=%zu hs=%zu", T, hs);
  return done(out, "attn_scores_bwd");
}
// The fused causal attention forward: P = softmax(Q K^T * scale + mask) and
// att = unheads(P @ V) [B*T, H*hs] from one kernel; *p_out receives P.
int64_t attn_fwd_impl(int64_t hq, int64_t hk, int64_t hv, int64_t hscale, size_t B, size_t T, size_t H, int64_t* p_out) {
  TensorBuffer *q = T_(hq), *kk = T_(hk), *v = T_(hv), *sc = T_(hscale);
  const size_t hs = q->shape[2], bh = B * H, C = H * hs;
  const size_t psh[3] = {bh, T, T}, osh[2] = {B * T, C};
  TensorBuffer* p = alloc_tensor(F32, psh, 3);
  TensorBuffer* out = alloc_tensor(F32, osh, 2);
  // P's tiles wholly above the diagonal stay unwritten: the fused VJP reads
  // only the others, and any other reader first has them filled with zeros
  if (!k::attn_fwd(q->f32(), kk->f32(), v->f32(), sc->f32(), nullptr, p->f32(), out->f32(), C, H, bh, T, hs, true,
                   stream(), /*full=*/false))
    fail("malus: attn_fwd: no fused kernel for t=%zu hs=%zu", T, hs);
  p->st->upper_unwritten_t = (uint32_t)T;
  const uint64_t seq = enqueue_mark("attn_fwd");
  p->write_seq = seq;
  out->write_seq = seq;
  *p_out = malus::H(p);
  return malus::H(out);
}
// dS of the fused causal attention and dQ = D + dS @ K from one kernel; *dq receives dQ.
int64_t attn_bwd_impl(int64_t hda, int64_t hv, int64_t hp, int64_t hscale, int64_t hk, const TensorBuffer* D,
                      int64_t* dq, size_t B, size_t T, size_t H) {
  TensorBuffer *da = T_(hda), *v = T_(hv), *p = T_(hp), *sc = T_(hscale), *kk = T_(hk);
  const size_t hs = v->shape[2], bh = B * H;
  const size_t sh[3] = {bh, T, T};
  TensorBuffer* out = alloc_tensor(F32, sh, 3);
  TensorBuffer* q = alloc_tensor(F32, kk->shape, 3);
  if (!k::attn_bwd(da->f32(), H * hs, H, v->f32(), p->f32(), sc->f32(), out->f32(), kk->f32(), q->f32(),
                   D ? D->f32() : nullptr, bh, T, hs, true, stream()))
    fail("malus: attn_bwd: no fused kernel for t=%zu hs=%zu", T, hs);
  const uint64_t seq = enqueue_mark("attn_bwd");
  out->write_seq = seq;
  q->write_seq = seq;
  *dq = malus::H(q);
  return malus::H(out);
}
// The whole attention VJP from one kernel: dS (scratch), dQ = Dq + dS @ K,
// dK = Dk + dS^T @ Q and dV = Dv + P^T @ dAtt, with dAtt [B*T, H*hs] read in
// place and Q, K, V, dQ, dK, dV [B*H, T, hs].
void attn_bwd_all_impl(int64_t hda, int64_t hq, int64_t hk, int64_t hv, int64_t hp, int64_t hscale,
                       const TensorBuffer* Dq, const TensorBuffer* Dk, const TensorBuffer* Dv, int64_t* dq, int64_t* dk,
                       int64_t* dv, size_t B, size_t T, size_t H) {
  TensorBuffer *da = T_(hda), *q = T_(hq), *kk = T_(hk), *v = T_(hv), *p = T_(hp), *sc = T_(hscale);
  const size_t hs = v->shape[2], bh = B * H;
  size_t bucket;
  float* ds = static_cast<float*>(pool_alloc(bh * T * T * sizeof(float), &bucket));
  TensorBuffer *oq = alloc_like(q), *ok = alloc_like(kk), *ov = alloc_like(v);
  const k::AttnKV kv{q->f32(), ok->f32(), Dk ? Dk->f32() : nullptr, ov->f32(), Dv ? Dv->f32() : nullptr};
  if (!k::attn_bwd(da->f32(), H * hs, H, v->f32(), p->f32(), sc->f32(), ds, kk->f32(), oq->f32(),
                   Dq ? Dq->f32() : nullptr, bh, T, hs, true, stream(), &kv, /*full=*/false))  // ds: scratch
    fail("malus: attn_bwd_all: no fused kernel for t=%zu hs=%zu", T, hs);
  pool_free(ds, bucket);  // stream order: later users of the buffer run after the kernel
  const uint64_t seq = enqueue_mark("attn_bwd_all");
  for (TensorBuffer* x : {oq, ok, ov}) x->write_seq = seq;
  *dq = malus::H(oq);
  *dk = malus::H(ok);
  *dv = malus::H(ov);
}
// Q, K and V all f32 (false) or all bf16 (true, the autocast storage policy:
// the kernels then run on the bf16 MFMA whatever the scope's state).
bool flash_qkv_bf16(const TensorBuffer* q, const TensorBuffer* kk, const TensorBuffer* v) {
  const int d = q->dtype;
  if ((d != F32 && d != BF16) || kk->dtype != d || v->dtype != d)
    fail("malus: flash attention: Q, K, V must be all f32 or all bf16 (dtype tags %d %d %d)", d, kk->dtype, v->dtype);
  return d == BF16;
}
// Flash attention of the model: Q, K, V [B*H, T, hs] -> att [B*T, H*hs]
// (causal); *lse_out [B*H, T].
int64_t flash_fwd_impl(int64_t hq, int64_t hk, int64_t hv, int64_t hscale, size_t B, size_t T, size_t H,
                       int64_t* lse_out) {
  TensorBuffer *q = T_(hq), *kk = T_(hk), *v = T_(hv), *sc = T_(hscale);
  const size_t hs = q->shape[2], bh = B * H, C = H * hs;
  const size_t lsh[2] = {bh, T}, osh[2] = {B * T, C};
  const bool s16 = flash_qkv_bf16(q, kk, v);
  TensorBuffer* lse = alloc_tensor(F32, lsh, 2);
  TensorBuffer* out = alloc_tensor(F32, osh, 2);
  if (!k::flash_fwd(q->f32(), kk->f32(), v->f32(), sc->f32(), out->f32(), C, H, lse->f32(), bh, T, hs, true,
                    k::autocast_on() || s16, stream(), s16))
    fail("malus: flash attention: no kernel for t=%zu hs=%zu", T, hs);
  const uint64_t seq = enqueue_mark("flash_attn_fwd");
  lse->write_seq = seq;
  out->write_seq = seq;
  *lse_out = malus::H(lse);
  return malus::H(out);
}
// Its VJP: dQ = Dq + ..., dK = Dk + ..., dV = Dv + ... from dAtt [B*T, H*hs].
void flash_bwd_impl(int64_t hda, int64_t hq, int64_t hk, int64_t hv, int64_t ho, int64_t hlse, int64_t hscale,
                    const TensorBuffer* Dq, const TensorBuffer* Dk, const TensorBuffer* Dv, int64_t* dq, int64_t* dk,
                    int64_t* dv, size_t B, size_t T, size_t H) {
  TensorBuffer *da = T_(hda), *q = T_(hq), *kk = T_(hk), *v = T_(hv), *o = T_(ho), *lse = T_(hlse), *sc = T_(hscale);
  const size_t hs = q->shape[2], bh = B * H, C = H * hs;
  const bool s16 = flash_qkv_bf16(q, kk, v);  // the gradients take Q, K, V's type
  if (s16 && (Dq || Dk || Dv)) fail("malus: flash attention VJP: bf16 gradients take no addends");
  TensorBuffer *oq = alloc_like(q), *ok = alloc_like(kk), *ov = alloc_like(v);
  size_t bucket;
  float* dsum = static_cast<float*>(pool_alloc(bh * T * sizeof(float), &bucket));
  const k::FlashBwd a{q->f32(), kk->f32(), v->f32(), o->f32(), da->f32(), lse->f32(), sc->f32(),
                      oq->f32(), ok->f32(), ov->f32(), dsum,
                      Dq ? Dq->f32() : nullptr, Dk ? Dk->f32() : nullptr, Dv ? Dv->f32() : nullptr};
  if (!k::flash_bwd(a, C, H, bh, T, hs, true, k::autocast_on() || s16, stream(), s16))
    fail("malus: flash attention VJP: no kernel for t=%zu hs=%zu", T, hs);
  pool_free(dsum, bucket);
  const uint64_t seq = enqueue_mark("flash_attn_bwd");
  for (TensorBuffer* x : {oq, ok, ov}) x->write_seq = seq;
  *dq = malus::H(oq);
  *dk = malus::H(ok);
  *dv = malus::H(ov);
}
// Scores S = Q @ K^T (the permute(K, 0, 2, 1) operand read in place): dQ = dS @ K, dK = dS^T @ Q  (+ D)
int64_t scores_bwd_q(int64_t hds, int64_t hk, const TensorBuffer* D, bool causal) {
  TensorBuffer *ds = T_(hds), *kk = T_(hk);
  const size_t bh = kk->shape[0], t = kk->shape[1], hs = kk->shape[2];
  if (!causal)
    return gemm_out(ds, kk, false, false, (int)bh, (int)t, (int)hs, (int)t, (long)(t * t), (long)(t * hs), kk->shape, 3, D);
  TensorBuffer* c = alloc_tensor(F32, kk->shape, 3);
  GemmLayouts L{dense_layout((long)t, (long)(t * t)), dense_layout((long)hs, (long)(t * hs)),
                dense_layout((long)hs, (long)(t * hs)), (int)ds->len, (int)kk->len, 1};
  return mapped(ds, kk, c, false, false, (int)bh, (int)t, (int)hs, (int)t, L, D, "scores_bwd_q");
}
// dK as the composed ops form it (nanogpt_modular.ml:54-57): the VJP of
// Q @ Kt with respect to Kt is Q^T @ dS [hs, t], permuted back to [t, hs].
// One GEMM with A = Q^T and B = dS writes that product through a transposed
// C layout (element (d, key) at key * hs + d), so the operands keep the
// composed GEMM's roles (the split-bf16 products depend on which operand is
// A).  Under a causal mask dS is zero above the diagonal and the full sum
// only adds exact zeros.
int64_t scores_bwd_k(int64_t hds, int64_t hq, const TensorBuffer* D, bool causal) {
  (void)causal;
  TensorBuffer *ds = T_(hds), *q = T_(hq);
  const size_t bh = q->shape[0], t = q->shape[1], hs = q->shape[2];
  TensorBuffer* c = alloc_tensor(F32, q->shape, 3);
  const GemmLayout ct{{0, 0, (int)(t * hs)}, {0, 0, 1}, {0, 0, (int)hs}};
  GemmLayouts L{dense_layout((long)hs, (long)(t * hs)), dense_layout((long)t, (long)(t * t)), ct, (int)q->len,
                (int)ds->len};
  return mapped(q, ds, c, true, false, (int)bh, (int)hs, (int)t, (int)t, L, D, "scores_bwd_k");
}

extern "C" {

int64_t tensor_matmul(int64_t ha, int64_t hb) {
  API_TRY
  return matmul_impl(ha, hb, nullptr);
  API_CATCH(0)
}
int64_t malus_std_matmul_bwd_a(int64_t ha, int64_t hb, int64_t hd) {
  API_TRY
  return matmul_bwd_a_impl(ha, hb, hd, nullptr);
  API_CATCH(0)
}
int64_t malus_std_matmul_bwd_b(int64_t ha, int64_t hb, int64_t hd) {
  API_TRY
  return matmul_bwd_b_impl(ha, hb, hd, nullptr);
  API_CATCH(0)
}

// ---- fused optimizer ------------------------------------------------------------------------
// examples/nanogpt_modular.ml:97-108 ("AdamW" with coupled L2).  Returns the
// new parameter; *m_out / *v_out receive the new moments.
int64_t malus_std_adam_l2(int64_t p, int64_t g, int64_t m, int64_t v, float lr, float b1, float b2, float eps, float wd,
                          int64_t t, int64_t* m_out, int64_t* v_out) {
  API_TRY
  TensorBuffer *tp = T(p), *tg = T(g), *tm = T(m), *tv = T(v);
  if (tg->len != tp->len || tm->len != tp->len || tv->len != tp->len) fail("malus: adam update: length mismatch");
  float bc1 = 1.0f - powf(b1, (float)t);  // `opt.beta1 ** t`: f32 powf (codegen-cpu/lib.rs:275)
  float bc2 = 1.0f - powf(b2, (float)t);
  TensorBuffer* po = alloc_like(tp);
  TensorBuffer* mo = alloc_like(tp);
  TensorBuffer* vo = alloc_like(tp);
  k::adam_l2(tp->f32(), tg->f32(), tm->f32(), tv->f32(), po->f32(), mo->f32(), vo->f32(), tp->len, lr, b1, b2,
             1.0f - b1, 1.0f - b2, bc1, bc2, eps, wd, stream());
  uint64_t seq = enqueue_mark("adam");
  po->write_seq = mo->write_seq = vo->write_seq = seq;
  *m_out = H(mo);
  *v_out = H(vo);
  return H(po);
  API_CATCH(0)
}

}  // extern "C"
