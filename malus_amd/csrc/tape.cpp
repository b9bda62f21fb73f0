// Define-by-run autograd tape: a C++ restatement of
// crates/malus-runtime/src/tape.rs (OpTag 14-79, BwdSlot 92-175, records
// 206-373, backward 421-729, grad registry 391-411 and 731-789).  The
// numbering of OpTag and BwdSlot is part of the ABI (the JIT emits the tags
// and registers slot pointers), so it is kept identical.  Every VJP runs
// through the registered slot function; by default the slots hold this
// library's stdlib host functions, and a JIT can overwrite them through
// tape_register_backward_fn exactly as compile_and_run does.
#include <cstdint>
#include <iterator>
#include <tuple>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "api.h"
#include "common.h"

extern "C" const char* malus_last_error(void);

namespace malus {
namespace {

enum OpTag : int32_t {
  Matmul = 0, Add = 1, Sub = 2, Mul = 3, Div = 4, Sigmoid = 5, Relu = 6, Tanh = 7, Exp = 8, Log = 9, Sqrt = 10,
  Abs = 11, Sum = 12, Transpose = 13, Neg = 14, ReduceSumAxis = 15, ReduceMeanAxis = 16, ReduceMaxAxis = 17,
  ReduceVarAxis = 18, Reshape = 19, Softmax = 20, Layernorm = 21, Gelu = 22, CrossEntropy = 23, Embedding = 24
};

// Fused nodes the library's own models record (never emitted by the JIT,
// so outside the reference's numbering).  Each stands for a chain of
// reference ops whose permutes are exact copies folded into GEMM
// addressing; its VJP computes the chain's gradients with the same values.
//   HeadProj (x, W) -> Qh:   reshape(permute(reshape(x @ W, B,T,H,hs), 0,2,1,3), B*H,T,hs)
//   Scores   (Q, K) -> S:    Q @ permute(K, 0,2,1)
//   AttnOut  (P, V) -> att:  reshape(permute(reshape(P @ V, B,H,T,hs), 0,2,1,3), B*T,C)
//   Attention (Q, K, V; P, scale) -> att: AttnOut(softmax(Scores(Q, K) * scale + causal mask), V),
//            with P the saved probabilities; the per-forward scale and mask
//            leaves are released before backward, so no gradient reaches them
//   LayerNormScale (x, w; y, var) -> out: layernorm(x, axis=-1) * w, with the
//            normalized rows y and the keepdim variance saved
//   GeluMatmul (h, W; ge) -> out: gelu(h) @ W, with ge = gelu(h) saved
//   FlashAttention (Q, K, V; att, lse, scale) -> att: Attention's value with an
//            online softmax (no P); the output and the row log-sum-exp are
//            saved for the VJP, which recomputes P
// meta holds {B, T, H} for HeadProj, AttnOut, Attention and FlashAttention.
enum FusedTag : int32_t {
  HeadProj = 100, Scores = 101, AttnOut = 102, Attention = 103, LayerNormScale = 104, GeluMatmul = 105,
  FlashAttention = 106
};

enum BwdSlot : int32_t {
  AddBwdA = 0, AddBwdB, SubBwdA, SubBwdB, MulBwdA, MulBwdB, DivBwdA, DivBwdB, SigmoidBwd, ReluBwd, TanhBwd, ExpBwd,
  LogBwd, SqrtBwd, AbsBwd, NegBwd, SumBwd, PermuteNdFwd, ReduceSumAxisBwd, ReduceMeanAxisBwd, ReduceMaxAxisBwd,
  ReduceVarAxisBwd, SoftmaxBwd, LayernormBwd, GeluBwd, CrossEntropyBwd, EmbeddingBwd, MatmulBwdA, MatmulBwdB, GradAcc,
  kNumSlots
};

struct TapeNode {
  int32_t op;
  std::vector<int64_t> saved;
  int64_t output;
  std::vector<int64_t> meta;
};

// Thread-local state, tape.rs:132-134 and 194-202.
thread_local bool t_recording = true;
thread_local std::vector<TapeNode> t_nodes;
thread_local std::unordered_set<int64_t> t_leaves;
thread_local std::unordered_map<int64_t, int64_t> t_leaf_grad;
thread_local size_t t_slots[kNumSlots] = {0};
thread_local bool t_slots_init = false;

void check_tag(int32_t tag) {
  if (tag < 0 || tag > Embedding) fail("malus: unknown op tag %d", tag);
}

void ensure_slots();

size_t slot(int32_t s) {
  ensure_slots();
  size_t p = t_slots[s];
  if (!p)
    fail("malus: backward kernel slot %d not registered - every stdlib backward fn must be registered before backward()", s);
  return p;
}

// A registered slot may be foreign code (the JIT's own VJP functions), and
// no C++ exception may cross it: the slot runs as an outermost call (any
// entry point it calls turns an error into a null handle and the last
// error), and a null result is raised here, in the tape's own frame.
struct SlotDepth {
  int saved;
  SlotDepth() : saved(g_api_depth) { g_api_depth = 0; }
  ~SlotDepth() { g_api_depth = saved; }
};

template <class F>
struct SlotCall;
template <class... A>
struct SlotCall<int64_t (*)(A...)> {
  int32_t s;
  int64_t (*f)(A...);
  int64_t operator()(A... a) const {
    int64_t r;
    {
      SlotDepth isolate;
      r = f(a...);
    }
    if (!r) fail("malus: the function in backward slot %d failed: %s", s, malus_last_error());
    return r;
  }
};

template <class F>
SlotCall<F> slot_fn(int32_t s) {
  return SlotCall<F>{s, reinterpret_cast<F>(slot(s))};
}

using Fn1 = int64_t (*)(int64_t);
using Fn2 = int64_t (*)(int64_t, int64_t);
using Fn3 = int64_t (*)(int64_t, int64_t, int64_t);
using Fn4 = int64_t (*)(int64_t, int64_t, int64_t, int64_t);
using FnNeg = int64_t (*)(int64_t, float);
using FnPerm = int64_t (*)(int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t, int64_t);

int64_t grad_acc(int64_t old_g, int64_t new_g) { return slot_fn<Fn2>(GradAcc)(old_g, new_g); }

thread_local bool t_fuse_vjps = true;  // fold GradAcc into matmul / layernorm VJP kernels

template <class F>
bool slot_is(int32_t s, F fn) { return t_fuse_vjps && slot(s) == reinterpret_cast<size_t>(fn); }

// Matmul VJP folded into the gradient accumulation: with the library's own
// MatmulBwd and GradAcc slots, grads[x] = old + dX comes out of one GEMM
// whose epilogue adds `old` (the product is rounded first, exactly as the
// GradAcc add of a separate result would round).  Accumulation order is the
// reference's: dA into grads[a], then dB into grads[b].
void accumulate_matmul(std::unordered_map<int64_t, int64_t>& grads, int64_t a, int64_t b, int64_t dout, bool need_a,
                       bool need_b) {
  auto fold = [&](int64_t x, bool is_a) {
    auto it = grads.find(x);
    const TensorBuffer* old = it == grads.end() ? nullptr : T(it->second);
    int64_t g = is_a ? matmul_bwd_a_impl(a, b, dout, old) : matmul_bwd_b_impl(a, b, dout, old);
    if (it == grads.end()) {
      grads.emplace(x, g);
    } else {
      release(T(it->second));
      it->second = g;
    }
  };
  if (need_a) fold(a, true);
  if (need_b) fold(b, false);
}

// A VJP that reads the values of a shape-only handle (the intermediate of a
// fused forward kernel) has no data to read: stop before any launch.
void need_values(int64_t h) {
  const TensorBuffer* t = T(h);
  if (t->len && (!t->st || !t->st->ptr))
    fail("malus: backward needs the values of a fused intermediate %s that was never stored", shape_str(t).c_str());
}

// Number of leading saved handles that are differentiable inputs.
int diff_inputs(int32_t op) {
  if (op == Attention || op == FlashAttention) return 3;
  if (op == Matmul || op == Add || op == Sub || op == Mul || op == Div || op == HeadProj || op == Scores ||
      op == AttnOut || op == LayerNormScale || op == GeluMatmul)
    return 2;
  return 1;
}

// grads[x] (+)= the VJP fn computes; with the library's GradAcc the old
// gradient rides into fn's GEMM epilogue as an addend (same rounding).
template <class F>
void fold_grad(std::unordered_map<int64_t, int64_t>& grads, int64_t x, F fn);

// Gradient liveness.  A gradient is computed only where it can reach a leaf
// the program still holds.  A registered leaf whose only references are the
// tape's own (the program released its handle before backward, like the
// per-forward `variable(...)` scale and mask of the attention block) can never
// be passed to tape_get_grad, and its registry entry is dropped by
// tape_on_release as soon as tape_clear lets go of it, so the VJPs that would
// only feed it are skipped.  Every gradient a live handle can observe is
// computed by the same kernels in the same order as without the pruning.
struct GradLiveness {
  std::unordered_map<int64_t, int64_t> refs;  // tape references per handle
  std::unordered_map<int64_t, bool> need;

  explicit GradLiveness(const std::vector<TapeNode>& nodes) {
    for (const TapeNode& n : nodes) {
      for (int64_t h : n.saved) ++refs[h];
      ++refs[n.output];
    }
    for (const TapeNode& n : nodes) {  // recording order: inputs precede the nodes that consume them
      bool any = false;
      for (int i = 0; i < diff_inputs(n.op); ++i) any = (*this)(n.saved[i]) || any;
      bool& o = need[n.output];
      o = o || any || live_leaf(n.output);
    }
  }
  bool live_leaf(int64_t h) const {
    if (!t_leaves.count(h)) return false;
    auto it = refs.find(h);
    return T(h)->rc.load() > (it == refs.end() ? 0 : it->second);
  }
  bool operator()(int64_t h) {
    auto it = need.find(h);
    if (it != need.end()) return it->second;
    const bool v = live_leaf(h);
    need.emplace(h, v);
    return v;
  }
};

// tape.rs:815-828: take ownership of new_grad, fold it into grads[input].
void accumulate(std::unordered_map<int64_t, int64_t>& grads, int64_t input, int64_t new_grad) {
  auto it = grads.find(input);
  if (it == grads.end()) {
    grads.emplace(input, new_grad);
    return;
  }
  int64_t old = it->second;
  int64_t summed = grad_acc(old, new_grad);
  release(T(old));
  release(T(new_grad));
  it->second = summed;
}

template <class F>
void fold_grad(std::unordered_map<int64_t, int64_t>& grads, int64_t x, F fn) {
  auto it = grads.find(x);
  if (!slot_is(GradAcc, &malus_std_broadcast_add_fwd)) {  // a JIT-registered GradAcc: call it
    accumulate(grads, x, fn(nullptr));
    return;
  }
  int64_t g = fn(it == grads.end() ? nullptr : T(it->second));
  if (it == grads.end()) {
    grads.emplace(x, g);
  } else {
    release(T(it->second));
    it->second = g;
  }
}

// normalize_perm / invert_perm (metal.rs:1275-1325)
std::vector<size_t> normalize_perm(const std::vector<size_t>& raw, size_t rank) {
  if (raw.empty()) {
    if (rank != 2) fail("malus: transpose() with no dim args requires a 2-D tensor, got rank %zu", rank);
    return {1, 0};
  }
  if (raw.size() == 2) {
    size_t i = raw[0], j = raw[1];
    if (i >= rank || j >= rank) fail("malus: transpose axis %zu or %zu out of range for rank-%zu tensor", i, j, rank);
    std::vector<size_t> p(rank);
    for (size_t k = 0; k < rank; ++k) p[k] = k;
    std::swap(p[i], p[j]);
    return p;
  }
  if (raw.size() == rank) {
    std::vector<bool> seen(rank, false);
    for (size_t p : raw) {
      if (p >= rank) fail("malus: permute dim %zu out of range for rank-%zu tensor", p, rank);
      if (seen[p]) fail("malus: permute has duplicate dim %zu", p);
      seen[p] = true;
    }
    return raw;
  }
  fail("malus: permute/transpose got %zu dim args for rank-%zu tensor; expected 0 (reverse 2-D), 2 (swap two axes), or %zu "
       "(full permute)",
       raw.size(), rank, rank);
}

int64_t permute_nd(int64_t h, const std::vector<size_t>& perm) {
  if (perm.size() > 8) fail("malus: permute supports rank <= 8, got rank %zu", perm.size());
  int64_t p[8] = {0};
  for (size_t i = 0; i < perm.size(); ++i) p[i] = (int64_t)perm[i];
  return slot_fn<FnPerm>(PermuteNdFwd)(h, p[0], p[1], p[2], p[3], p[4], p[5], p[6], p[7]);
}

}  // namespace

std::vector<size_t> tape_normalize_perm(const std::vector<size_t>& raw, size_t rank) { return normalize_perm(raw, rank); }

void tape_on_release(int64_t handle) {
  // tape.rs:783-789
  auto it = t_leaf_grad.find(handle);
  int64_t g = 0;
  if (it != t_leaf_grad.end()) {
    g = it->second;
    t_leaf_grad.erase(it);
  }
  t_leaves.erase(handle);
  if (g) release(T(g));
}

namespace {
void ensure_slots() {
  if (t_slots_init) return;
  t_slots_init = true;
  auto reg = [](int32_t s, auto fn) { if (!t_slots[s]) t_slots[s] = reinterpret_cast<size_t>(fn); };
  reg(AddBwdA, &malus_std_add_bwd_a);
  reg(AddBwdB, &malus_std_add_bwd_b);
  reg(SubBwdA, &malus_std_sub_bwd_a);
  reg(SubBwdB, &malus_std_sub_bwd_b);
  reg(MulBwdA, &malus_std_mul_bwd_a);
  reg(MulBwdB, &malus_std_mul_bwd_b);
  reg(DivBwdA, &malus_std_div_bwd_a);
  reg(DivBwdB, &malus_std_div_bwd_b);
  reg(SigmoidBwd, &malus_std_sigmoid_bwd);
  reg(ReluBwd, &malus_std_relu_bwd);
  reg(TanhBwd, &malus_std_tanh_bwd);
  reg(ExpBwd, &malus_std_broadcast_mul_fwd);  // BWD_SLOT_FNS (codegen-cpu/lib.rs:201): dout * e
  reg(LogBwd, &malus_std_broadcast_div_fwd);  // dout / x
  reg(SqrtBwd, &malus_std_sqrt_bwd);
  reg(AbsBwd, &malus_std_abs_bwd);
  reg(NegBwd, &malus_std_scale_fwd);
  reg(SumBwd, &malus_std_sum_bwd);
  reg(PermuteNdFwd, &malus_std_permute_nd_fwd);
  reg(ReduceSumAxisBwd, &malus_std_reduce_sum_axis_bwd);
  reg(ReduceMeanAxisBwd, &malus_std_reduce_mean_axis_bwd);
  reg(ReduceMaxAxisBwd, &malus_std_reduce_max_axis_bwd);
  reg(ReduceVarAxisBwd, &malus_std_reduce_var_axis_bwd);
  reg(SoftmaxBwd, &malus_std_softmax_bwd);
  reg(LayernormBwd, &malus_std_layernorm_bwd);
  reg(GeluBwd, &malus_std_gelu_bwd);
  reg(CrossEntropyBwd, &malus_std_cross_entropy_bwd);
  reg(EmbeddingBwd, &malus_std_embedding_bwd);
  reg(MatmulBwdA, &malus_std_matmul_bwd_a);
  reg(MatmulBwdB, &malus_std_matmul_bwd_b);
  reg(GradAcc, &malus_std_broadcast_add_fwd);  // codegen-cpu/lib.rs:219
}
}  // namespace

void register_default_backward_fns() { ensure_slots(); }

}  // namespace malus

using namespace malus;

namespace malus {
void tape_record_fused(int32_t op, const std::vector<int64_t>& saved, int64_t out, const std::vector<int64_t>& meta) {
  if (!t_recording) return;
  const size_t want = op == FlashAttention ? 6 : op == Attention ? 5 : op == LayerNormScale ? 4
                                               : op == GeluMatmul ? 3 : 2;
  if (op < HeadProj || op > FlashAttention) fail("malus: unknown fused op tag %d", op);
  if (saved.size() != want) fail("malus: fused op %d takes %zu saved handles, got %zu", op, want, saved.size());
  for (int64_t h : saved) retain(T(h));
  retain(T(out));
  t_nodes.push_back({op, saved, out, meta});
}
}  // namespace malus

extern "C" {

// 1 (default): fold gradient accumulation into the matmul and layernorm VJP
// kernels when the library's own slots are registered; 0: separate GradAcc
// adds.  Values are the same either way (testing and comparison knob).
void malus_tape_set_fused_vjps(int on) { t_fuse_vjps = on != 0; }

void tape_register_backward_fn(int32_t s, size_t fnptr) {
  API_TRY
  if (s < 0 || s >= kNumSlots) fail("malus: backward slot %d out of range", s);
  ensure_slots();
  t_slots[s] = fnptr;
  API_CATCH()
}

size_t malus_tape_backward_fn(int32_t s) {
  if (s < 0 || s >= kNumSlots) return 0;
  ensure_slots();
  return t_slots[s];
}

void tape_record_binop(int32_t op, int64_t a, int64_t b, int64_t out) {
  API_TRY
  if (!t_recording) return;
  check_tag(op);
  retain(T(a)); retain(T(b)); retain(T(out));
  t_nodes.push_back({op, {a, b}, out, {}});
  API_CATCH()
}

void tape_record_unary(int32_t op, int64_t x, int64_t out) {
  API_TRY
  if (!t_recording) return;
  check_tag(op);
  retain(T(x)); retain(T(out));
  t_nodes.push_back({op, {x}, out, {}});
  API_CATCH()
}

void tape_record_reduce(int32_t op, int64_t x, int64_t out, int64_t axis, int64_t keepdim) {
  API_TRY
  if (!t_recording) return;
  check_tag(op);
  retain(T(x)); retain(T(out));
  t_nodes.push_back({op, {x}, out, {axis, keepdim}});
  API_CATCH()
}

void tape_record_perm(int32_t op, int64_t x, int64_t out, const size_t* dims, size_t ndims) {
  API_TRY
  if (!t_recording) return;
  check_tag(op);
  retain(T(x)); retain(T(out));
  std::vector<int64_t> meta;
  if (dims && ndims)
    for (size_t i = 0; i < ndims; ++i) meta.push_back((int64_t)dims[i]);
  t_nodes.push_back({op, {x}, out, meta});
  API_CATCH()
}

// var_h: ownership transferred from the caller (tape.rs:289-310)
void tape_record_layernorm(int32_t op, int64_t x, int64_t out, int64_t var_h, int64_t axis) {
  API_TRY
  if (!t_recording) { release(T(var_h)); return; }
  check_tag(op);
  retain(T(x)); retain(T(out));
  t_nodes.push_back({op, {x, var_h}, out, {axis}});
  API_CATCH()
}

// softmax_h: ownership transferred (tape.rs:312-337)
void tape_record_cross_entropy(int32_t op, int64_t logits, int64_t out, int64_t softmax_h, int64_t targets) {
  API_TRY
  if (!t_recording) { release(T(softmax_h)); return; }
  check_tag(op);
  retain(T(logits)); retain(T(out)); retain(T(targets));
  t_nodes.push_back({op, {logits, softmax_h, targets}, out, {}});
  API_CATCH()
}

void tape_record_embedding(int32_t op, int64_t weight, int64_t indices, int64_t out) {
  API_TRY
  if (!t_recording) return;
  check_tag(op);
  retain(T(weight)); retain(T(indices)); retain(T(out));
  t_nodes.push_back({op, {weight, indices}, out, {}});
  API_CATCH()
}

void tape_register_leaf(int64_t h) { t_leaves.insert(h); }

void tape_pause(void) { t_recording = false; }
void tape_resume(void) { t_recording = true; }

void tape_clear(void) {
  API_TRY
  std::vector<TapeNode> nodes;
  nodes.swap(t_nodes);
  for (auto& n : nodes) {
    for (int64_t h : n.saved) release(T(h));
    release(T(n.output));
  }
  API_CATCH()
}

int64_t tape_get_grad(int64_t h) {
  API_TRY
  auto it = t_leaf_grad.find(h);
  if (it != t_leaf_grad.end()) {
    retain(T(it->second));
    return it->second;
  }
  TensorBuffer* t = T(h);
  TensorBuffer* z = alloc_tensor(F32, t->shape, t->ndim);
  k::fill(z->f32(), 0.0f, z->len, stream());
  z->write_seq = enqueue_mark("zeros_like");
  return H(z);
  API_CATCH(0)
}

size_t malus_tape_len(void) { return t_nodes.size(); }
void malus_tape_registry_lens(size_t* out2) { out2[0] = t_leaves.size(); out2[1] = t_leaf_grad.size(); }

// tape.rs:421-729
void backward(int64_t loss) {
  API_TRY
  std::vector<TapeNode> nodes = t_nodes;  // snapshot
  std::unordered_map<int64_t, int64_t> grads;
  {
    TensorBuffer* lt = T(loss);
    TensorBuffer* seed = alloc_tensor(F32, lt->shape, lt->ndim);
    k::fill(seed->f32(), 1.0f, seed->len, stream());
    seed->write_seq = enqueue_mark("seed");
    grads.emplace(loss, H(seed));
  }
  GradLiveness need(nodes);
  // A layernorm scale whose weight is a live leaf that no other record
  // reads gets its weight gradient only at the leaf fold below, so the
  // column combines of those gradients are queued and run in one launch
  // before it (the same sums per column); the guard runs them if backward
  // stops early.
  std::unordered_map<int64_t, int> reads;
  for (const TapeNode& n : nodes)
    for (int64_t h : n.saved) ++reads[h];
  std::vector<int64_t> deferred;  // gradients whose combine is queued
  struct FlushGuard {
    ~FlushGuard() {
      try {
        k::col_combine_flush(stream());
      } catch (...) {
      }
    }
  } flush_guard;
  for (auto it = nodes.rbegin(); it != nodes.rend(); ++it) {
    const TapeNode& n = *it;
    auto g = grads.find(n.output);
    if (g == grads.end()) continue;
    const int64_t dout = g->second;
    const int ni = diff_inputs(n.op);
    const bool na = need(n.saved[0]);
    const bool nb = ni > 1 && need(n.saved[1]);
    const bool nc = ni > 2 && need(n.saved[2]);
    if (!na && !nb && !nc) continue;
    if (n.op == HeadProj && std::distance(it, nodes.rend()) >= 3) {
      // The q, k, v projections of one input sit back to back on the tape:
      // run their three VJPs as one grouped launch each for dx (accumulated
      // in this same order) and for the three dW (same values as one node
      // at a time).
      const TapeNode &n1 = *(it + 1), &n2 = *(it + 2);
      const int64_t x = n.saved[0];
      auto g1 = grads.find(n1.output), g2 = grads.find(n2.output);
      const bool grouped = n1.op == HeadProj && n2.op == HeadProj && n1.saved[0] == x && n2.saved[0] == x &&
                           n1.meta == n.meta && n2.meta == n.meta && g1 != grads.end() && g2 != grads.end() && na &&
                           need(n.saved[1]) && need(n1.saved[1]) && need(n2.saved[1]) && !grads.count(n.saved[1]) &&
                           !grads.count(n1.saved[1]) && !grads.count(n2.saved[1]) &&
                           slot_is(GradAcc, &malus_std_broadcast_add_fwd);
      if (grouped) {
        const int64_t dq[3] = {dout, g1->second, g2->second};
        const int64_t w[3] = {n.saved[1], n1.saved[1], n2.saved[1]};
        for (int64_t h : w) need_values(h);
        need_values(x);
        const size_t Bm = (size_t)n.meta[0], Tm = (size_t)n.meta[1], Hm = (size_t)n.meta[2];
        fold_grad(grads, x, [&](const TensorBuffer* o) { return head_proj_bwd_x3(dq, w, Bm, Tm, Hm, o); });
        int64_t dw[3];
        head_proj_bwd_w3(x, dq, Bm, Tm, Hm, dw);
        for (int i = 0; i < 3; ++i) grads.emplace(w[i], dw[i]);
        it += 2;
        continue;
      }
    }
    if (n.op == Embedding && std::distance(it, nodes.rend()) >= 2 && na &&
        slot_is(EmbeddingBwd, &malus_std_embedding_bwd)) {
      // The token and position embeddings of one sum sit back to back on
      // the tape with one gradient: both VJPs from one list launch and one
      // sum launch, accumulated in this same order.
      const TapeNode& n1 = *(it + 1);
      auto g1 = grads.find(n1.output);
      int64_t dwa = 0, dwb = 0;
      if (n1.op == Embedding && g1 != grads.end() && g1->second == dout && need(n1.saved[0]) &&
          n1.saved[0] != n.saved[0] &&
          embedding_bwd2_impl(n.saved[0], n.saved[1], n1.saved[0], n1.saved[1], dout, &dwa, &dwb)) {
        accumulate(grads, n.saved[0], dwa);
        accumulate(grads, n1.saved[0], dwb);
        ++it;
        continue;
      }
    }
    switch (n.op) {
      case Matmul: {
        int64_t a = n.saved[0], b = n.saved[1];
        if (na) need_values(b);
        if (nb) need_values(a);
        if (slot_is(MatmulBwdA, &malus_std_matmul_bwd_a) && slot_is(MatmulBwdB, &malus_std_matmul_bwd_b) &&
            slot_is(GradAcc, &malus_std_broadcast_add_fwd)) {
          accumulate_matmul(grads, a, b, dout, na, nb);
          break;
        }
        if (na) accumulate(grads, a, slot_fn<Fn3>(MatmulBwdA)(a, b, dout));
        if (nb) accumulate(grads, b, slot_fn<Fn3>(MatmulBwdB)(a, b, dout));
        break;
      }
      case Attention: {  // saved {Q, K, V, P, scale}
        const int64_t q = n.saved[0], kk = n.saved[1], v = n.saved[2], pr = n.saved[3], sc = n.saved[4];
        const size_t Bm = (size_t)n.meta[0], Tm = (size_t)n.meta[1], Hm = (size_t)n.meta[2];
        for (int64_t h : n.saved) need_values(h);
        if (na && nb && nc && q != kk && q != v && kk != v && slot_is(GradAcc, &malus_std_broadcast_add_fwd)) {
          // all four products from one kernel; each gradient folds into its
          // own entry, in the order below (dV, dQ, dK)
          auto old = [&](int64_t x) -> const TensorBuffer* {
            auto f = grads.find(x);
            return f == grads.end() ? nullptr : T(f->second);
          };
          int64_t dq = 0, dk = 0, dv = 0;
          attn_bwd_all_impl(dout, q, kk, v, pr, sc, old(q), old(kk), old(v), &dq, &dk, &dv, Bm, Tm, Hm);
          for (auto [x, g] : {std::pair{v, dv}, std::pair{q, dq}, std::pair{kk, dk}}) {
            auto f = grads.find(x);
            if (f == grads.end()) {
              grads.emplace(x, g);
            } else {
              release(T(f->second));
              f->second = g;
            }
          }
          break;
        }
        // AttnOut's VJP (dP, dV), the softmax and scale VJPs, then Scores' (dQ, dK);
        // the GEMMs read P whole
        materialize_upper_tiles(T(pr));
        if (nc) fold_grad(grads, v, [&](const TensorBuffer* o) { return attn_out_bwd_v(pr, dout, Bm, Tm, Hm, o, true); });
        if (na || nb) {
          int64_t ds = 0;
          if (na) {  // dS and dQ = dS @ K from one kernel
            fold_grad(grads, q, [&](const TensorBuffer* o) {
              int64_t dq = 0;
              ds = attn_bwd_impl(dout, v, pr, sc, kk, o, &dq, Bm, Tm, Hm);
              return dq;
            });
          } else {
            ds = attn_scores_bwd_impl(dout, v, pr, sc, Bm, Tm, Hm);
          }
          if (nb) fold_grad(grads, kk, [&](const TensorBuffer* o) { return scores_bwd_k(ds, q, o, true); });
          release(T(ds));
        }
        break;
      }
      case FlashAttention: {  // saved {Q, K, V, att, lse, scale}: the three gradients from two kernels
        const int64_t q = n.saved[0], kk = n.saved[1], v = n.saved[2], o = n.saved[3], lse = n.saved[4],
                      sc = n.saved[5];
        const size_t Bm = (size_t)n.meta[0], Tm = (size_t)n.meta[1], Hm = (size_t)n.meta[2];
        for (int64_t h : n.saved) need_values(h);
        // with the library's GradAcc an existing gradient rides into the
        // kernels as an addend and the result replaces it (same rounding)
        const bool fold = q != kk && q != v && kk != v && slot_is(GradAcc, &malus_std_broadcast_add_fwd);
        auto old = [&](int64_t x) -> const TensorBuffer* {
          auto f = grads.find(x);
          return fold && f != grads.end() ? T(f->second) : nullptr;
        };
        int64_t dq = 0, dk = 0, dv = 0;
        flash_bwd_impl(dout, q, kk, v, o, lse, sc, old(q), old(kk), old(v), &dq, &dk, &dv, Bm, Tm, Hm);
        for (auto [x, gr, needed] : {std::tuple{v, dv, nc}, std::tuple{q, dq, na}, std::tuple{kk, dk, nb}}) {
          auto f = grads.find(x);
          if (!needed) {
            release(T(gr));
          } else if (fold && f != grads.end()) {
            release(T(f->second));
            f->second = gr;
          } else {
            accumulate(grads, x, gr);
          }
        }
        break;
      }
      case GeluMatmul: {  // saved {h, W, ge}: the matmul's VJPs (dge, then dW), then the GELU VJP of dge
        const int64_t h = n.saved[0], w = n.saved[1], ge = n.saved[2];
        need_values(h);
        need_values(w);
        need_values(ge);
        // a bf16 gelu(h) comes from the autocast storage policy, whose h has
        // this node as its one reader: dh is then read by bf16 GEMMs only
        const bool dh_bf16 = T(ge)->dtype == BF16;
        if (na) fold_grad(grads, h, [&](const TensorBuffer* o) { return gelu_matmul_bwd_h(dout, w, h, o, dh_bf16 && !o); });
        if (nb) fold_grad(grads, w, [&](const TensorBuffer* o) { return matmul_bwd_b_impl(ge, w, dout, o); });
        break;
      }
      case LayerNormScale: {  // saved {x, w, y, var}
        const int64_t x = n.saved[0], w = n.saved[1], y = n.saved[2], var = n.saved[3];
        need_values(w);
        need_values(y);
        // the multiply's VJPs (dy, then dw), then the layernorm VJP of dy
        if (na && nb && slot_is(MulBwdB, &malus_std_mul_bwd_b)) {  // both from one row kernel where it applies
          int64_t dw = 0;
          const bool defer_dw = reads[w] == 1 && t_leaves.count(w) && !grads.count(w);
          fold_grad(grads, x, [&](const TensorBuffer* o) {
            const int64_t dx = ln_affine_bwd_xw(y, var, w, dout, o, &dw, defer_dw);
            return dx ? dx : ln_affine_bwd_x(y, var, w, dout, o);
          });
          if (dw && defer_dw) deferred.push_back(dw);
          accumulate(grads, w, dw ? dw : slot_fn<Fn3>(MulBwdB)(dout, y, w));
          break;
        }
        if (nb) accumulate(grads, w, slot_fn<Fn3>(MulBwdB)(dout, y, w));
        if (na) fold_grad(grads, x, [&](const TensorBuffer* o) { return ln_affine_bwd_x(y, var, w, dout, o); });
        break;
      }
      case HeadProj: case Scores: case AttnOut: {
        const int64_t a = n.saved[0], b = n.saved[1];
        if (na) need_values(b);
        if (nb) need_values(a);
        const size_t Bm = n.meta.empty() ? 0 : (size_t)n.meta[0], Tm = n.meta.empty() ? 0 : (size_t)n.meta[1],
                     Hm = n.meta.empty() ? 0 : (size_t)n.meta[2];
        if (n.op == HeadProj) {
          if (na) fold_grad(grads, a, [&](const TensorBuffer* o) { return head_proj_bwd_x(dout, b, Bm, Tm, Hm, o); });
          if (nb) fold_grad(grads, b, [&](const TensorBuffer* o) { return head_proj_bwd_w(a, dout, Bm, Tm, Hm, o); });
        } else if (n.op == Scores) {
          if (na) fold_grad(grads, a, [&](const TensorBuffer* o) { return scores_bwd_q(dout, b, o, false); });
          if (nb) fold_grad(grads, b, [&](const TensorBuffer* o) { return scores_bwd_k(dout, a, o, false); });
        } else {
          if (na) fold_grad(grads, a, [&](const TensorBuffer* o) { return attn_out_bwd_p(dout, b, Bm, Tm, Hm, o); });
          if (nb) fold_grad(grads, b, [&](const TensorBuffer* o) { return attn_out_bwd_v(a, dout, Bm, Tm, Hm, o, false); });
        }
        break;
      }
      case Add: case Sub: {
        int64_t a = n.saved[0], b = n.saved[1];
        int32_t sa = n.op == Add ? AddBwdA : SubBwdA, sb = n.op == Add ? AddBwdB : SubBwdB;
        if (na) accumulate(grads, a, slot_fn<Fn2>(sa)(dout, a));
        if (nb) accumulate(grads, b, slot_fn<Fn2>(sb)(dout, b));
        break;
      }
      case Mul: case Div: {
        int64_t a = n.saved[0], b = n.saved[1];
        int32_t sa = n.op == Mul ? MulBwdA : DivBwdA, sb = n.op == Mul ? MulBwdB : DivBwdB;
        if (na) need_values(b);
        if (nb) { need_values(a); need_values(b); }
        if (na) accumulate(grads, a, slot_fn<Fn3>(sa)(dout, a, b));
        if (nb) accumulate(grads, b, slot_fn<Fn3>(sb)(dout, a, b));
        break;
      }
      case Sigmoid: accumulate(grads, n.saved[0], slot_fn<Fn2>(SigmoidBwd)(n.output, dout)); break;
      case Relu: accumulate(grads, n.saved[0], slot_fn<Fn2>(ReluBwd)(n.saved[0], dout)); break;
      case Tanh: accumulate(grads, n.saved[0], slot_fn<Fn2>(TanhBwd)(n.output, dout)); break;
      case Exp: accumulate(grads, n.saved[0], slot_fn<Fn2>(ExpBwd)(dout, n.output)); break;
      case Log: accumulate(grads, n.saved[0], slot_fn<Fn2>(LogBwd)(dout, n.saved[0])); break;
      case Sqrt: accumulate(grads, n.saved[0], slot_fn<Fn2>(SqrtBwd)(n.output, dout)); break;
      case Abs: accumulate(grads, n.saved[0], slot_fn<Fn2>(AbsBwd)(n.saved[0], dout)); break;
      case Sum: accumulate(grads, n.saved[0], slot_fn<Fn2>(SumBwd)(n.saved[0], dout)); break;
      case Transpose: {
        int64_t x = n.saved[0];
        std::vector<size_t> raw;
        for (int64_t v : n.meta) raw.push_back((size_t)v);
        std::vector<size_t> perm = normalize_perm(raw, (size_t)T(x)->ndim);
        std::vector<size_t> inv(perm.size());
        for (size_t i = 0; i < perm.size(); ++i) inv[perm[i]] = i;
        accumulate(grads, x, permute_nd(dout, inv));
        break;
      }
      case Reshape: {
        int64_t x = n.saved[0];
        accumulate(grads, x, H(make_alias(T(dout), T(x)->shape, T(x)->ndim)));
        break;
      }
      case Neg: accumulate(grads, n.saved[0], slot_fn<FnNeg>(NegBwd)(dout, -1.0f)); break;
      case ReduceSumAxis: accumulate(grads, n.saved[0], slot_fn<Fn3>(ReduceSumAxisBwd)(n.saved[0], dout, n.meta[0])); break;
      case ReduceMeanAxis: accumulate(grads, n.saved[0], slot_fn<Fn3>(ReduceMeanAxisBwd)(n.saved[0], dout, n.meta[0])); break;
      case ReduceMaxAxis:
        accumulate(grads, n.saved[0], slot_fn<Fn4>(ReduceMaxAxisBwd)(n.saved[0], n.output, dout, n.meta[0]));
        break;
      case ReduceVarAxis: accumulate(grads, n.saved[0], slot_fn<Fn3>(ReduceVarAxisBwd)(n.saved[0], dout, n.meta[0])); break;
      case Softmax: accumulate(grads, n.saved[0], slot_fn<Fn3>(SoftmaxBwd)(n.output, dout, n.meta[0])); break;
      case Layernorm:
        if (slot_is(LayernormBwd, &malus_std_layernorm_bwd) && slot_is(GradAcc, &malus_std_broadcast_add_fwd)) {
          // grads[x] = old + dx from one kernel (same rounding as GradAcc)
          auto it = grads.find(n.saved[0]);
          const TensorBuffer* old = it == grads.end() ? nullptr : T(it->second);
          int64_t g = layernorm_bwd_impl(n.output, n.saved[1], dout, n.meta[0], old);
          if (it == grads.end()) {
            grads.emplace(n.saved[0], g);
          } else {
            release(T(it->second));
            it->second = g;
          }
          break;
        }
        accumulate(grads, n.saved[0], slot_fn<Fn4>(LayernormBwd)(n.output, n.saved[1], dout, n.meta[0]));
        break;
      case Gelu: accumulate(grads, n.saved[0], slot_fn<Fn2>(GeluBwd)(n.saved[0], dout)); break;
      case CrossEntropy:
        accumulate(grads, n.saved[0], slot_fn<Fn3>(CrossEntropyBwd)(n.saved[1], n.saved[2], dout));
        break;
      case Embedding: accumulate(grads, n.saved[0], slot_fn<Fn3>(EmbeddingBwd)(n.saved[0], n.saved[1], dout)); break;
      default: fail("malus: backward: unhandled op tag %d", n.op);
    }
  }
  k::col_combine_flush(stream());
  if (!deferred.empty()) {  // host reads of those gradients wait for the combine
    const uint64_t seq = enqueue_mark("layernorm scale gradients");
    for (int64_t h : deferred) T(h)->write_seq = seq;
  }
  // fold leaf grads into the persistent registry (tape.rs:694-721)
  std::vector<int64_t> to_release;
  for (int64_t leaf : t_leaves) {
    auto g = grads.find(leaf);
    if (g == grads.end()) continue;
    int64_t new_g = g->second;
    grads.erase(g);
    auto old = t_leaf_grad.find(leaf);
    if (old == t_leaf_grad.end()) {
      t_leaf_grad.emplace(leaf, new_g);
    } else {
      int64_t summed = grad_acc(old->second, new_g);
      to_release.push_back(old->second);
      to_release.push_back(new_g);
      old->second = summed;
    }
  }
  for (int64_t h : to_release) release(T(h));
  for (auto& kv : grads) release(T(kv.second));
  tape_clear();
  API_CATCH()
}

void tape_reset(void) {
  API_TRY
  t_leaves.clear();
  std::vector<int64_t> gs;
  for (auto& kv : t_leaf_grad) gs.push_back(kv.second);
  t_leaf_grad.clear();
  for (int64_t g : gs) release(T(g));
  tape_clear();
  t_recording = true;
  API_CATCH()
}

void tape_zero_grad(const int64_t* handles, size_t count) {
  API_TRY
  if (!handles || !count) return;
  std::vector<int64_t> rel;
  for (size_t i = 0; i < count; ++i) {
    auto it = t_leaf_grad.find(handles[i]);
    if (it != t_leaf_grad.end()) {
      rel.push_back(it->second);
      t_leaf_grad.erase(it);
    }
  }
  for (int64_t g : rel) release(T(g));
  API_CATCH()
}

}  // extern "C"
