// kernel_dispatch / kernel_dispatch_v2 and runtime_init: the binding ABI a
// JIT'd malus program uses for kernel launches (metal.rs:1860-2065,
// metal.rs:304-336).
//
// runtime_init receives id -> kernel source.  Two kinds of source arrive:
//   * a stdlib or synthesized builtin kernel, which the HIP emitter tags with
//     a first line "//@malus-builtin <kernel name>".  Its id is bound to a
//     hand-written gfx950 implementation of that kernel's semantics; the
//     launch's grid x tg is read as the logical iteration space, and the
//     implementation picks its own geometry (no 1024-thread cap, coalesced
//     loads) -- the override rule of the build;
//   * any other (user) kernel: HIP C++ compiled once with hipRTC for the
//     device's gfx target and cached by source text with the id normalized
//     away, like the pipeline cache of metal.rs:300-336.
//
// Launch ABI of user kernels (what the emitter generates):
//   v1: malus_kernel_<id>(const T* in0, ..., T* out, unsigned n)
//       launched over n = out.len threads in 256-thread blocks;
//   v2: malus_kernel_<id>(const T* in0, ..., T* out[, Uniforms u],
//                         TensorMeta in0_meta, ..., TensorMeta out_meta)
//       launched with the caller's grid (workgroup counts) and tg.
#include <hip/hip_runtime.h>
#include <hip/hiprtc.h>

#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "api.h"
#include "common.h"

using namespace malus;

namespace {

enum class Builtin {
  None,
  // v2 stdlib kernels
  BcastAdd, BcastSub, BcastMul, BcastDiv,
  ReduceSum, ReduceMean, ReduceMax, ReduceVar,
  Softmax, Layernorm, LayernormVar, Gelu, CeNll, Embedding,
  Transpose2d, Permute3d, PermuteNd, Scale, FillLike, Eq,
  SigmoidBwd, ReluBwd, TanhBwd, SqrtBwd, AbsBwd, ExpandAxis, RsqrtEps, GeluBwd, CeBwd, EmbeddingBwd,
  // v1 synthesized builtins
  Add, Sub, Mul, Div, AddS, SubS, MulS, DivS, RSubS, RDivS,
  Relu, Sigmoid, Tanh, Exp, Log, Sqrt, Abs,
};

const std::unordered_map<std::string, Builtin>& builtin_names() {
  static const std::unordered_map<std::string, Builtin> m = {
      {"__broadcast_add_kernel", Builtin::BcastAdd}, {"__broadcast_sub_kernel", Builtin::BcastSub},
      {"__broadcast_mul_kernel", Builtin::BcastMul}, {"__broadcast_div_kernel", Builtin::BcastDiv},
      {"__reduce_sum_kernel", Builtin::ReduceSum}, {"__reduce_mean_kernel", Builtin::ReduceMean},
      {"__reduce_max_kernel", Builtin::ReduceMax}, {"__reduce_var_kernel", Builtin::ReduceVar},
      {"__softmax_kernel", Builtin::Softmax}, {"__layernorm_kernel", Builtin::Layernorm},
      {"__layernorm_var_kernel", Builtin::LayernormVar}, {"__gelu_kernel", Builtin::Gelu},
      {"__cross_entropy_nll_kernel", Builtin::CeNll}, {"__embedding_kernel", Builtin::Embedding},
      {"__transpose_2d_kernel", Builtin::Transpose2d}, {"__permute_3d_kernel", Builtin::Permute3d},
      {"__permute_nd_kernel", Builtin::PermuteNd}, {"__scale_kernel", Builtin::Scale},
      {"__fill_like_kernel", Builtin::FillLike}, {"__eq_kernel", Builtin::Eq},
      {"__sigmoid_bwd_kernel", Builtin::SigmoidBwd}, {"__relu_bwd_kernel", Builtin::ReluBwd},
      {"__tanh_bwd_kernel", Builtin::TanhBwd}, {"__sqrt_bwd_kernel", Builtin::SqrtBwd},
      {"__abs_bwd_kernel", Builtin::AbsBwd}, {"__expand_axis_kernel", Builtin::ExpandAxis},
      {"__rsqrt_eps_kernel", Builtin::RsqrtEps}, {"__gelu_bwd_kernel", Builtin::GeluBwd},
      {"__cross_entropy_bwd_kernel", Builtin::CeBwd}, {"__embedding_bwd_kernel", Builtin::EmbeddingBwd},
      {"malus_add", Builtin::Add}, {"malus_sub", Builtin::Sub}, {"malus_mul", Builtin::Mul},
      {"malus_div", Builtin::Div}, {"malus_add_scalar", Builtin::AddS}, {"malus_sub_scalar", Builtin::SubS},
      {"malus_mul_scalar", Builtin::MulS}, {"malus_div_scalar", Builtin::DivS},
      {"malus_rsub_scalar", Builtin::RSubS}, {"malus_rdiv_scalar", Builtin::RDivS},
      {"relu", Builtin::Relu}, {"sigmoid", Builtin::Sigmoid}, {"tanh", Builtin::Tanh}, {"exp", Builtin::Exp},
      {"log", Builtin::Log}, {"sqrt", Builtin::Sqrt}, {"abs", Builtin::Abs},
  };
  return m;
}

struct KernelEntry {
  Builtin builtin = Builtin::None;
  hipModule_t module = nullptr;
  hipFunction_t fn = nullptr;
  // From the emitter's annotations: v1 inputs read only at [0] (bit i =
  // input i), and the v2 uniforms blob size (-1: unknown).
  uint32_t scalar_inputs = 0;
  long uniform_bytes = -1;
  // v1: element bytes of the output, then of each input, as the kernel
  // declares them (empty: not annotated).
  std::vector<long> elem_bytes;
};

// The emitter's "//@malus-<key> <value>" annotation lines.
// A list annotation "//@malus-<key> v0 v1 ...": the numbers up to the line's end.
std::vector<long> annotation_list(const std::string& src, const char* key) {
  std::vector<long> out;
  std::string tag = std::string("//@malus-") + key + " ";
  size_t p = src.find(tag);
  if (p == std::string::npos) return out;
  const char* c = src.c_str() + p + tag.size();
  while (*c && *c != '\n') {
    char* end = nullptr;
    long v = strtol(c, &end, 10);
    if (end == c) break;
    out.push_back(v);
    c = end;
  }
  return out;
}

bool annotation(const std::string& src, const char* key, long* value) {
  std::string tag = std::string("//@malus-") + key + " ";
  size_t p = src.find(tag);
  if (p == std::string::npos) return false;
  *value = strtol(src.c_str() + p + tag.size(), nullptr, 10);
  return true;
}

struct Registry {
  std::mutex mu;
  std::unordered_map<uint64_t, KernelEntry> by_id;
  std::unordered_map<std::string, std::pair<hipModule_t, std::string>> by_source;  // normalized source -> module
};

Registry& reg() {
  static Registry r;
  return r;
}

std::string device_arch() {
  hipDeviceProp_t p;
  int dev;
  MALUS_HIP(hipGetDevice(&dev));
  MALUS_HIP(hipGetDeviceProperties(&p, dev));
  std::string a = p.gcnArchName;
  size_t c = a.find(':');
  return c == std::string::npos ? a : a.substr(0, c);
}

// Source-cache key: the text with the kernel id taken out of every name the
// emitter derives from it (malus_kernel_<id>, Uniforms_<id>), so identical
// bodies registered under different ids share one module (metal.rs:304-336).
std::string normalize(uint64_t id, const std::string& src) {
  std::string s = src;
  for (const std::string& prefix : {std::string("malus_kernel_"), std::string("Uniforms_")}) {
    const std::string needle = prefix + std::to_string(id);
    for (size_t pos = s.find(needle); pos != std::string::npos; pos = s.find(needle, pos + prefix.size() + 1)) {
      const size_t end = pos + needle.size();
      if (end < s.size() && isdigit((unsigned char)s[end])) continue;  // a longer id
      s.replace(pos, needle.size(), prefix + "X");
    }
  }
  return s;
}

// Options for every runtime-compiled kernel: the same code generation rules as
// the library's own translation units (no FMA contraction, denormals kept, and
// no packed-FP32 instruction selection).
std::vector<std::string> rtc_options(const std::string& arch) {
  return {"--offload-arch=" + arch, "-O3", "-std=c++17", "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
}

// hipRTC: source -> code object for `arch`.  Needs no device.  On failure the
// log goes to *log and an empty vector is returned.
std::vector<char> rtc_compile(const std::string& src, const std::string& name, const std::string& arch,
                              std::string* log) {
  hiprtcProgram prog;
  if (hiprtcCreateProgram(&prog, src.c_str(), name.c_str(), 0, nullptr, nullptr) != HIPRTC_SUCCESS) {
    if (log) *log = "hiprtcCreateProgram failed";
    return {};
  }
  std::vector<std::string> opts = rtc_options(arch);
  std::vector<const char*> argv;
  for (const std::string& o : opts) argv.push_back(o.c_str());
  hiprtcResult r = hiprtcCompileProgram(prog, (int)argv.size(), argv.data());
  size_t log_size = 0;
  hiprtcGetProgramLogSize(prog, &log_size);
  std::string text(log_size, '\0');
  if (log_size) hiprtcGetProgramLog(prog, &text[0]);
  while (!text.empty() && text.back() == '\0') text.pop_back();
  if (r != HIPRTC_SUCCESS) {
    hiprtcDestroyProgram(&prog);
    if (log) *log = std::string(hiprtcGetErrorString(r)) + "\n" + text;
    return {};
  }
  size_t code_size = 0;
  hiprtcGetCodeSize(prog, &code_size);
  std::vector<char> code(code_size);
  hiprtcGetCode(prog, code.data());
  hiprtcDestroyProgram(&prog);
  if (log) *log = text;
  return code;
}

hipModule_t compile_hiprtc(uint64_t id, const std::string& src) {
  std::string name = "malus_kernel_" + std::to_string(id) + ".hip";
  std::string log;
  std::vector<char> code = rtc_compile(src, name, device_arch(), &log);
  if (code.empty())
    fail("malus: HIP compilation failed for kernel %llu: %s", (unsigned long long)id, log.c_str());
  hipModule_t mod;
  MALUS_HIP(hipModuleLoadData(&mod, code.data()));
  return mod;
}

struct TensorMeta {  // the v2 binding's per-tensor metadata (metal.rs:2017-2048)
  uint32_t ndim;
  uint32_t shape[8];
  uint32_t strides[8];
};

TensorMeta meta_of(const TensorBuffer* t) {
  TensorMeta m{};
  int rank = t->ndim < 8 ? t->ndim : 8;
  m.ndim = (uint32_t)rank;
  size_t stride = 1;
  for (int k = rank - 1; k >= 0; --k) {
    m.shape[k] = (uint32_t)t->shape[k];
    m.strides[k] = (uint32_t)stride;
    stride *= t->shape[k];
  }
  return m;
}

int32_t u_i32(const void* u, size_t bytes, int idx) {
  if ((size_t)(idx + 1) * 4 > bytes) fail("malus: kernel_dispatch_v2: uniforms blob too small (%zu bytes) for field %d", bytes, idx);
  int32_t v;
  memcpy(&v, static_cast<const uint8_t*>(u) + 4 * idx, 4);
  return v;
}
float u_f32(const void* u, size_t bytes, int idx) {
  if ((size_t)(idx + 1) * 4 > bytes) fail("malus: kernel_dispatch_v2: uniforms blob too small (%zu bytes) for field %d", bytes, idx);
  float v;
  memcpy(&v, static_cast<const uint8_t*>(u) + 4 * idx, 4);
  return v;
}

void need_inputs(const std::vector<TensorBuffer*>& in, size_t n, const char* what) {
  if (in.size() < n) fail("malus: builtin kernel %s expects %zu tensor inputs, got %zu", what, n, in.size());
}

void need_len(const TensorBuffer* t, size_t n, const char* what) {
  if (t->len < n) fail("malus: builtin kernel %s reads %zu elements from a %zu-element tensor", what, n, t->len);
}

// ref kernel semantics of __broadcast_<op>_kernel: out (A's shape) = a[flat] op b[b_flat]
void bcast_kernel(int op, TensorBuffer* a, TensorBuffer* b, TensorBuffer* out) {
  if (out->len != a->len) fail("malus: __broadcast kernel output length %zu != input length %zu", out->len, a->len);
  if (b->ndim > a->ndim) fail("malus: __broadcast kernel expects a.ndim >= b.ndim");
  k::BcastDesc d{};
  d.ndim = a->ndim;
  const int off = a->ndim - b->ndim;
  size_t as = 1;
  size_t bstr[kMaxRank];
  size_t bs = 1;
  for (int i = b->ndim - 1; i >= 0; --i) { bstr[i] = bs; bs *= b->shape[i]; }
  for (int i = a->ndim - 1; i >= 0; --i) {
    d.out_shape[i] = (uint32_t)a->shape[i];
    d.p_stride[i] = (uint32_t)as;
    as *= a->shape[i];
    int db = i - off;
    size_t bdim = db >= 0 ? b->shape[db] : 1;
    if (bdim > 1 && bdim < a->shape[i])
      fail("malus: broadcast shape mismatch: %s vs %s", shape_str(a).c_str(), shape_str(b).c_str());
    d.q_stride[i] = bdim > 1 ? (uint32_t)bstr[db] : 0u;
  }
  if (a->len == 0) return;
  k::binary_general(op, a->f32(), b->f32(), out->f32(), a->len, d, stream());
}

void run_builtin_v2(Builtin b, std::vector<TensorBuffer*>& in, TensorBuffer* out, const size_t* grid, const void* u,
                    size_t ub) {
  hipStream_t s = stream();
  const size_t groups = grid[0] * grid[1] * grid[2];
  switch (b) {
    case Builtin::BcastAdd: need_inputs(in, 2, "__broadcast_add_kernel"); bcast_kernel(k::ADD, in[0], in[1], out); break;
    case Builtin::BcastSub: need_inputs(in, 2, "__broadcast_sub_kernel"); bcast_kernel(k::SUB, in[0], in[1], out); break;
    case Builtin::BcastMul: need_inputs(in, 2, "__broadcast_mul_kernel"); bcast_kernel(k::MUL, in[0], in[1], out); break;
    case Builtin::BcastDiv: need_inputs(in, 2, "__broadcast_div_kernel"); bcast_kernel(k::DIV, in[0], in[1], out); break;
    case Builtin::ReduceSum: case Builtin::ReduceMean: case Builtin::ReduceMax: case Builtin::ReduceVar: {
      need_inputs(in, 1, "__reduce_*_kernel");
      size_t axis = (size_t)u_i32(u, ub, 0), inner = (size_t)u_i32(u, ub, 1);
      if (inner == 0) fail("malus: reduce kernel with inner == 0");
      size_t outer = groups / inner;
      need_len(in[0], outer * axis * inner, "__reduce_*_kernel");
      need_len(out, outer * inner, "__reduce_*_kernel (output)");
      int op = b == Builtin::ReduceSum ? k::R_SUM : b == Builtin::ReduceMean ? k::R_MEAN : b == Builtin::ReduceMax ? k::R_MAX : k::R_VAR;
      k::reduce_axis(op, in[0]->f32(), out->f32(), outer, axis, inner, s);
      break;
    }
    case Builtin::Softmax: case Builtin::Layernorm: case Builtin::LayernormVar: {
      need_inputs(in, 1, "__softmax/layernorm kernel");
      size_t axis = (size_t)u_i32(u, ub, 0), inner = (size_t)u_i32(u, ub, 1);
      if (inner == 0) fail("malus: row kernel with inner == 0");
      size_t outer = groups / inner;
      need_len(in[0], outer * axis * inner, "__softmax/layernorm kernel");
      need_len(out, outer * axis * inner, "__softmax/layernorm kernel (output)");
      if (b == Builtin::Softmax) {
        k::softmax(in[0]->f32(), out->f32(), outer, axis, inner, s);
      } else {
        float eps = u_f32(u, ub, 2);
        size_t bucket, bucket2;
        float* var = static_cast<float*>(pool_alloc(outer * inner * sizeof(float), &bucket));
        if (b == Builtin::Layernorm) {
          k::layernorm(in[0]->f32(), out->f32(), var, outer, axis, inner, eps, s);
        } else {  // variance broadcast over the full input shape (layernorm.ml:35-57)
          float* y = static_cast<float*>(pool_alloc(outer * axis * inner * sizeof(float), &bucket2));
          k::layernorm(in[0]->f32(), y, var, outer, axis, inner, eps, s);
          k::expand_axis(var, out->f32(), outer, axis, inner, s);
          pool_free(y, bucket2);
        }
        pool_free(var, bucket);
      }
      break;
    }
    case Builtin::Gelu: need_inputs(in, 1, "__gelu_kernel"); need_len(in[0], out->len, "__gelu_kernel"); k::unary(k::GELU, in[0]->f32(), out->f32(), out->len, s); break;
    case Builtin::CeNll: {
      need_inputs(in, 2, "__cross_entropy_nll_kernel");
      size_t v = (size_t)u_i32(u, ub, 0), n = out->len;
      need_len(in[0], n * v, "__cross_entropy_nll_kernel");
      need_len(in[1], n, "__cross_entropy_nll_kernel (targets)");
      if (in[1]->dtype != I32) fail("malus: cross-entropy targets must be Tensor<i32>");
      k::nll_gather(in[0]->f32(), in[1]->i32(), out->f32(), n, v, device_error_flag(), s);
      break;
    }
    case Builtin::Embedding: {
      need_inputs(in, 2, "__embedding_kernel");
      size_t d = (size_t)u_i32(u, ub, 0);
      if (d == 0 || in[1]->dtype != I32) fail("malus: __embedding_kernel needs embed_dim > 0 and Tensor<i32> indices");
      size_t t = out->len / d;
      need_len(in[1], t, "__embedding_kernel (indices)");
      k::embedding(in[0]->f32(), in[1]->i32(), out->f32(), t, in[0]->len / d, d, device_error_flag(), s);
      break;
    }
    case Builtin::Transpose2d: {
      need_inputs(in, 1, "__transpose_2d_kernel");
      size_t perm[2] = {1, 0};
      if (in[0]->ndim != 2) fail("malus: __transpose_2d_kernel expects a 2-D input");
      k::permute(in[0]->f32(), out->f32(), 2, in[0]->shape, perm, s);
      break;
    }
    case Builtin::Permute3d: case Builtin::PermuteNd: {
      need_inputs(in, 1, "__permute kernel");
      TensorBuffer* x = in[0];
      int nd = x->ndim;
      if (b == Builtin::Permute3d && nd != 3) fail("malus: __permute_3d_kernel expects a 3-D input");
      size_t perm[kMaxRank];
      std::vector<bool> seen((size_t)nd, false);
      for (int i = 0; i < nd; ++i) {
        int32_t p = u_i32(u, ub, i);
        if (p < 0 || p >= nd || seen[(size_t)p]) fail("malus: invalid permutation entry %d for rank %d", p, nd);
        seen[(size_t)p] = true;
        perm[i] = (size_t)p;
      }
      need_len(out, x->len, "__permute kernel (output)");
      k::permute(x->f32(), out->f32(), nd, x->shape, perm, s);
      break;
    }
    case Builtin::Scale: need_inputs(in, 1, "__scale_kernel"); need_len(in[0], out->len, "__scale_kernel"); k::binary_scalar(k::MUL, in[0]->f32(), nullptr, u_f32(u, ub, 0), true, out->f32(), out->len, s); break;
    case Builtin::FillLike: k::fill(out->f32(), u_f32(u, ub, 0), out->len, s); break;
    case Builtin::Eq: need_inputs(in, 2, "__eq_kernel"); need_len(in[0], out->len, "__eq_kernel"); need_len(in[1], out->len, "__eq_kernel"); k::eq(in[0]->f32(), in[1]->f32(), out->f32(), out->len, s); break;
    case Builtin::SigmoidBwd: case Builtin::ReluBwd: case Builtin::TanhBwd: case Builtin::SqrtBwd: case Builtin::AbsBwd:
    case Builtin::GeluBwd: {
      need_inputs(in, 2, "unary VJP kernel");
      need_len(in[0], out->len, "unary VJP kernel");
      need_len(in[1], out->len, "unary VJP kernel");
      int op = b == Builtin::SigmoidBwd ? k::B_SIGMOID : b == Builtin::ReluBwd ? k::B_RELU : b == Builtin::TanhBwd ? k::B_TANH
             : b == Builtin::SqrtBwd ? k::B_SQRT : b == Builtin::AbsBwd ? k::B_ABS : k::B_GELU;
      k::unary_bwd(op, in[0]->f32(), in[1]->f32(), out->f32(), out->len, s);
      break;
    }
    case Builtin::ExpandAxis: {
      need_inputs(in, 1, "__expand_axis_kernel");
      size_t axis = (size_t)u_i32(u, ub, 0), inner = (size_t)u_i32(u, ub, 1);
      if (axis == 0 || inner == 0) fail("malus: __expand_axis_kernel with an empty axis");
      size_t outer = out->len / (axis * inner);
      need_len(in[0], outer * inner, "__expand_axis_kernel");
      k::expand_axis(in[0]->f32(), out->f32(), outer, axis, inner, s);
      break;
    }
    case Builtin::RsqrtEps: need_inputs(in, 1, "__rsqrt_eps_kernel"); need_len(in[0], out->len, "__rsqrt_eps_kernel"); k::rsqrt_eps(in[0]->f32(), u_f32(u, ub, 0), out->f32(), out->len, s); break;
    case Builtin::CeBwd: {
      need_inputs(in, 2, "__cross_entropy_bwd_kernel");
      size_t v = (size_t)u_i32(u, ub, 0);
      float scale = u_f32(u, ub, 1);
      if (v == 0 || in[1]->dtype != I32) fail("malus: __cross_entropy_bwd_kernel needs vocab > 0 and Tensor<i32> targets");
      size_t n = out->len / v;
      need_len(in[0], n * v, "__cross_entropy_bwd_kernel");
      need_len(in[1], n, "__cross_entropy_bwd_kernel (targets)");
      k::ce_bwd(in[0]->f32(), in[1]->i32(), nullptr, scale, out->f32(), n, v, s);
      break;
    }
    case Builtin::EmbeddingBwd: {
      need_inputs(in, 2, "__embedding_bwd_kernel");
      size_t t = (size_t)u_i32(u, ub, 0), d = (size_t)u_i32(u, ub, 1);
      if (d == 0 || in[1]->dtype != I32) fail("malus: __embedding_bwd_kernel needs embed_dim > 0 and Tensor<i32> indices");
      need_len(in[0], t * d, "__embedding_bwd_kernel");
      need_len(in[1], t, "__embedding_bwd_kernel (indices)");
      k::embedding_bwd(in[0]->f32(), in[1]->i32(), out->f32(), t, out->len / d, d, s);
      break;
    }
    default: fail("malus: builtin kernel is not a kernel_dispatch_v2 kernel");
  }
}

void run_builtin_v1(Builtin b, std::vector<TensorBuffer*>& in, TensorBuffer* out) {
  hipStream_t s = stream();
  const size_t n = out->len;
  // the synthesized builtins are f32 kernels (codegen-gpu/lib.rs:373-418)
  for (TensorBuffer* t : in)
    if (t->dtype != F32) fail("malus: kernel_dispatch: the builtin kernels take f32 tensors (got dtype tag %d)", t->dtype);
  auto same = [&](int op) {
    need_inputs(in, 2, "elementwise builtin");
    need_len(in[1], n, "elementwise builtin");
    k::binary_same(op, in[0]->f32(), in[1]->f32(), out->f32(), n, s);
  };
  auto scal = [&](int op, bool right) {
    need_inputs(in, 2, "scalar builtin");
    need_len(in[1], 1, "scalar builtin");
    k::binary_scalar(op, in[0]->f32(), in[1]->f32(), 0.0f, right, out->f32(), n, s);
  };
  switch (b) {
    case Builtin::Add: same(k::ADD); break;
    case Builtin::Sub: same(k::SUB); break;
    case Builtin::Mul: same(k::MUL); break;
    case Builtin::Div: same(k::DIV); break;
    case Builtin::AddS: scal(k::ADD, true); break;
    case Builtin::SubS: scal(k::SUB, true); break;
    case Builtin::MulS: scal(k::MUL, true); break;
    case Builtin::DivS: scal(k::DIV, true); break;
    case Builtin::RSubS: scal(k::SUB, false); break;
    case Builtin::RDivS: scal(k::DIV, false); break;
    case Builtin::Relu: k::unary(k::RELU, in[0]->f32(), out->f32(), n, s); break;
    case Builtin::Sigmoid: k::unary(k::SIGMOID, in[0]->f32(), out->f32(), n, s); break;
    case Builtin::Tanh: k::unary(k::TANH, in[0]->f32(), out->f32(), n, s); break;
    case Builtin::Exp: k::unary(k::EXP, in[0]->f32(), out->f32(), n, s); break;
    case Builtin::Log: k::unary(k::LOG, in[0]->f32(), out->f32(), n, s); break;
    case Builtin::Sqrt: k::unary(k::SQRT, in[0]->f32(), out->f32(), n, s); break;
    case Builtin::Abs: k::unary(k::ABS, in[0]->f32(), out->f32(), n, s); break;
    default: fail("malus: builtin kernel is not a kernel_dispatch (v1) kernel");
  }
}

KernelEntry lookup(uint64_t id, const char* api) {
  std::lock_guard<std::mutex> lk(reg().mu);
  auto it = reg().by_id.find(id);
  if (it == reg().by_id.end()) fail("malus: %s: kernel_id %llu not registered", api, (unsigned long long)id);
  return it->second;
}

}  // namespace

namespace malus {
bool dispatch_has_builtin(const std::string& name) { return builtin_names().count(name) != 0; }
}  // namespace malus

extern "C" {

// runtime_init(&HashMap<u64, String>) as a C ABI (metal.rs:304-336).
void malus_runtime_init(const uint64_t* ids, const char* const* sources, size_t n) {
  API_TRY
  ensure_init();
  for (size_t i = 0; i < n; ++i) {
    std::string src = sources[i];
    KernelEntry e;
    const std::string tag = "//@malus-builtin ";
    size_t p = src.find(tag);
    if (p != std::string::npos) {
      size_t b = p + tag.size(), end = src.find_first_of(" \r\n", b);
      std::string name = src.substr(b, end == std::string::npos ? std::string::npos : end - b);
      auto it = builtin_names().find(name);
      if (it == builtin_names().end()) fail("malus: unknown builtin kernel tag '%s'", name.c_str());
      e.builtin = it->second;
    } else {
      // byte-identical bodies compiled under another id reuse that module
      // and that id's entry-point name
      std::string key = normalize(ids[i], src);
      std::lock_guard<std::mutex> lk(reg().mu);
      auto it = reg().by_source.find(key);
      std::string fname;
      if (it != reg().by_source.end()) {
        e.module = it->second.first;
        fname = it->second.second;
      } else {
        e.module = compile_hiprtc(ids[i], src);
        fname = "malus_kernel_" + std::to_string(ids[i]);
        reg().by_source.emplace(key, std::make_pair(e.module, fname));
      }
      if (hipModuleGetFunction(&e.fn, e.module, fname.c_str()) != hipSuccess)
        fail("malus: kernel function '%s' not found", fname.c_str());
      long v;
      if (annotation(src, "v1-scalar-inputs", &v) && v >= 0 && v < 32) e.scalar_inputs |= 1u << v;
      if (annotation(src, "v2-uniform-bytes", &v)) e.uniform_bytes = v;
      e.elem_bytes = annotation_list(src, "v1-elem-bytes");
    }
    std::lock_guard<std::mutex> lk(reg().mu);
    reg().by_id[ids[i]] = e;
  }
  API_CATCH()
}

// Compile HIP source for `arch` (e.g. "gfx950") with the options runtime_init
// uses, without a device.  Returns the code object's size (0 on failure, with
// the compiler log in `log`); the object is copied to `code` when cap allows.
size_t malus_rtc_compile(const char* src, const char* arch, void* code, size_t cap, char* log, size_t log_cap) {
  std::string text;
  std::vector<char> obj = rtc_compile(src ? src : "", "malus_rtc.hip", arch ? arch : "gfx950", &text);
  if (log && log_cap) {
    size_t n = std::min(text.size(), log_cap - 1);
    memcpy(log, text.data(), n);
    log[n] = '\0';
  }
  if (code && cap >= obj.size()) memcpy(code, obj.data(), obj.size());
  return obj.size();
}

int malus_kernel_is_builtin(uint64_t id) {
  std::lock_guard<std::mutex> lk(reg().mu);
  auto it = reg().by_id.find(id);
  return it != reg().by_id.end() && it->second.builtin != Builtin::None;
}

int64_t kernel_dispatch(uint64_t id, const int64_t* handles, size_t count) {
  API_TRY
  if (count < 1 || !handles) fail("malus: kernel_dispatch requires at least one input handle");
  KernelEntry e = lookup(id, "kernel_dispatch");
  std::vector<TensorBuffer*> in;
  for (size_t i = 0; i < count; ++i) in.push_back(T(handles[i]));
  for (TensorBuffer* t : in) materialize_upper_tiles(t);
  // output: dtype and shape of inputs[0] (metal.rs:1878-1888)
  TensorBuffer* out = alloc_tensor(in[0]->dtype, in[0]->shape, in[0]->ndim);
  if (out->len == 0) return H(out);
  if (e.builtin != Builtin::None) {
    run_builtin_v1(e.builtin, in, out);
  } else {
    // The output takes input 0's dtype (metal.rs:1878-1888); the kernel
    // reads and writes the element widths it declares, so they must agree.
    if (!e.elem_bytes.empty()) {
      if (e.elem_bytes.size() != in.size() + 1)
        fail("malus: kernel_dispatch: kernel %llu takes %zu tensor inputs, got %zu", (unsigned long long)id,
             e.elem_bytes.size() - 1, in.size());
      if ((long)dtype_size(out->dtype) != e.elem_bytes[0])
        fail("malus: kernel_dispatch: kernel %llu writes %ld-byte elements, but its output takes input 0's dtype "
             "(%zu-byte elements)", (unsigned long long)id, e.elem_bytes[0], dtype_size(out->dtype));
      for (size_t i = 0; i < in.size(); ++i)
        if ((long)dtype_size(in[i]->dtype) != e.elem_bytes[i + 1])
          fail("malus: kernel_dispatch: kernel %llu reads input %zu as %ld-byte elements, got %zu-byte elements",
               (unsigned long long)id, i, e.elem_bytes[i + 1], dtype_size(in[i]->dtype));
    }
    // an emitted implicit-map kernel reads in_i[tid] for every tid < out.len
    // (a scalar-broadcast builtin reads its scalar input at [0] only)
    for (size_t i = 0; i < in.size(); ++i) {
      const size_t need = (i < 32 && (e.scalar_inputs >> i) & 1u) ? 1 : out->len;
      if (in[i]->len < need)
        fail("malus: kernel_dispatch input of %zu elements is shorter than the %zu elements the kernel reads",
             in[i]->len, need);
    }
    std::vector<void*> ptrs;
    for (auto* t : in) ptrs.push_back(t->data());
    ptrs.push_back(out->data());
    unsigned n = (unsigned)out->len;
    std::vector<void*> args;
    for (auto& p : ptrs) args.push_back(&p);
    args.push_back(&n);
    unsigned blocks = (n + 255) / 256;
    MALUS_HIP(hipModuleLaunchKernel(e.fn, blocks, 1, 1, 256, 1, 1, 0, stream(), args.data(), nullptr));
  }
  out->write_seq = enqueue_mark("kernel_dispatch");
  return H(out);
  API_CATCH(0)
}

int64_t kernel_dispatch_v2(uint64_t id, const int64_t* handles, size_t hc, const size_t* grid, const size_t* tg,
                           const size_t* out_shape, size_t out_ndim, int32_t out_dtype, const void* uniforms,
                           size_t ubytes) {
  API_TRY
  if (!grid) fail("malus: kernel_dispatch_v2 grid_dims must not be null");
  if (!tg) fail("malus: kernel_dispatch_v2 tg_dims must not be null");
  KernelEntry e = lookup(id, "kernel_dispatch_v2");
  std::vector<TensorBuffer*> in;
  for (size_t i = 0; i < hc; ++i) in.push_back(T(handles[i]));
  for (TensorBuffer* t : in) {  // an explicit kernel may write its tensor arguments
    materialize_upper_tiles(t);
    if (t->st) t->st->causal_t = t->st->causal_mask_t = 0;
  }
  TensorBuffer* out;
  if (out_ndim == 0) {  // inherit input 0's shape; dtype from the tag or input 0 (metal.rs:1973-1981)
    if (in.empty()) fail("malus: kernel_dispatch_v2: out_ndim==0 but no tensor inputs");
    out = alloc_tensor(out_dtype >= 0 ? out_dtype : in[0]->dtype, in[0]->shape, in[0]->ndim);
  } else {
    out = alloc_tensor(out_dtype, out_shape, (int)out_ndim);
  }
  if (out->len == 0) return H(out);
  if (e.builtin != Builtin::None) {
    run_builtin_v2(e.builtin, in, out, grid, uniforms, ubytes);
  } else {
    std::vector<void*> ptrs;
    for (auto* t : in) ptrs.push_back(t->data());
    ptrs.push_back(out->data());
    std::vector<TensorMeta> metas;
    for (auto* t : in) metas.push_back(meta_of(t));
    metas.push_back(meta_of(out));
    if (e.uniform_bytes >= 0 && (size_t)e.uniform_bytes != ubytes)
      fail("malus: kernel_dispatch_v2: kernel %llu takes %ld bytes of uniforms, got %zu", (unsigned long long)id,
           e.uniform_bytes, ubytes);
    std::vector<uint8_t> ublob(ubytes);
    if (ubytes && uniforms) memcpy(ublob.data(), uniforms, ubytes);
    std::vector<void*> args;
    for (auto& p : ptrs) args.push_back(&p);
    if (ubytes) args.push_back(ublob.data());
    for (auto& m : metas) args.push_back(&m);
    for (int d = 0; d < 3; ++d)
      if (grid[d] == 0 || tg[d] == 0) fail("malus: kernel_dispatch_v2: zero grid or threadgroup dimension");
    if (tg[0] * tg[1] * tg[2] > 1024) fail("malus: kernel_dispatch_v2: threadgroup of %zu threads exceeds 1024", tg[0] * tg[1] * tg[2]);
    MALUS_HIP(hipModuleLaunchKernel(e.fn, (unsigned)grid[0], (unsigned)grid[1], (unsigned)grid[2], (unsigned)tg[0],
                                    (unsigned)tg[1], (unsigned)tg[2], 0, stream(), args.data(), nullptr));
  }
  out->write_seq = enqueue_mark("kernel_dispatch_v2");
  return H(out);
  API_CATCH(0)
}

}  // extern "C"
