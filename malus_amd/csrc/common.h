// Shared runtime types for libmalus_hip: tensor handles, the device pool,
// stream ordering, error reporting, and the host-side launch wrappers of
// every hand-written gfx950 kernel.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

namespace malus {

// ---- dtype tags (metal.rs:26-50; the numbering is part of the ABI) ----------
enum Dtype : int32_t {
  F32 = 0, F16 = 1, BF16 = 2, I8 = 3, I16 = 4, I32 = 5, I64 = 6,
  U8 = 7, U16 = 8, U32 = 9, U64 = 10
};
size_t dtype_size(int32_t tag);  // aborts on unknown tags

constexpr int kMaxRank = 8;

// Device allocation shared by a tensor and its reshape aliases
// (metal.rs:262-276 PoolState + the MTLBuffer it guards).
struct Storage {
  void* ptr = nullptr;
  size_t bytes = 0;              // bucketed allocation size
  std::atomic<int> aliases{0};   // TensorBuffers referencing this storage
  // t > 0: holds attention probabilities [.., t, t] written by a causal
  // attention forward (zero above the diagonal); reset by any host write
  // and by a kernel_dispatch_v2 that receives the tensor.
  uint32_t causal_t = 0;
  // t > 0: holds tensor_causal_mask(t) (0 on and below the diagonal, -1e9
  // above), as built by it or verified once; reset like causal_t.
  uint32_t causal_mask_t = 0;
  // t > 0: causal attention probabilities [.., t, t] whose 32 x 32 tiles
  // wholly above the diagonal were never written (the fused backward reads
  // only the tiles on and below it); attn_zero_upper_tiles fills them.
  uint32_t upper_unwritten_t = 0;
};

// One tensor handle (metal.rs:280-296 TensorBuffer).  The i64 handle the ABI
// passes around is a TensorBuffer*.
struct TensorBuffer {
  Storage* st = nullptr;
  int32_t dtype = F32;
  size_t len = 0;
  int ndim = 0;
  size_t shape[kMaxRank] = {0};
  std::atomic<int64_t> rc{1};
  uint64_t write_seq = 0;        // stream sequence of the last GPU write (0 = ready)
  // A bf16 copy of this tensor's values for bf16 GEMM operands (the
  // autocast storage policy keeps one per weight matrix; this holds a
  // reference).  It stands for this tensor while copy->copy_of == this and
  // copy->copy_seq == write_seq: refreshed after the tensor's last write.
  // With split f32 products the model keeps a split copy in this slot
  // instead (split3): the three bf16 pieces of every value, h, m and l, as
  // three planes of the tensor's layout one after another.
  TensorBuffer* bf16_copy = nullptr;
  const TensorBuffer* copy_of = nullptr;  // on a copy: the tensor it was last refreshed from
  uint64_t copy_seq = 0;                  // ... and that tensor's write_seq at the refresh
  bool split3 = false;                    // on a copy: the three-plane split form

  float* f32() const { return static_cast<float*>(st->ptr); }
  int32_t* i32() const { return static_cast<int32_t*>(st->ptr); }
  void* data() const { return st->ptr; }
  size_t bytes() const { return len * dtype_size(dtype); }
};

inline TensorBuffer* T(int64_t h) { return reinterpret_cast<TensorBuffer*>(h); }
inline int64_t H(TensorBuffer* t) { return reinterpret_cast<int64_t>(t); }

// ---- errors (ADR-0006 panic-only model: "malus: ..." then abort) -----------
[[noreturn]] void fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void check_hip(hipError_t e, const char* what);
#define MALUS_HIP(x) ::malus::check_hip((x), #x)
std::string shape_str(const TensorBuffer* t);

// ---- context ---------------------------------------------------------------
void ensure_init();
// Set-up of the allocation-free entry point's scratch array on `device`
// (noalloc.hip); called once by ensure_init with that device current.
void noalloc_init_device(int device);
hipStream_t stream();
// Marks one enqueued GPU operation; returns its sequence number.  Every op
// that writes a tensor stamps that tensor's write_seq with it.
uint64_t enqueue_mark(const char* op_name);
void flush_if_pending(TensorBuffer* t);   // metal.rs:244-252
void sync_all();                          // gpu_barrier body

// ---- allocation ------------------------------------------------------------
// Allocate an uninitialized tensor (kernels must write every element).
TensorBuffer* alloc_tensor(int32_t dtype, const size_t* shape, int ndim);
TensorBuffer* alloc_like(const TensorBuffer* t);
TensorBuffer* alloc_f32(std::initializer_list<size_t> shape);
TensorBuffer* make_alias(TensorBuffer* src, const size_t* shape, int ndim);  // reshape_to
// A handle with shape and dtype but no device storage: the tape node of an
// intermediate a fused kernel keeps in registers (only its shape is ever
// consulted).  Host reads of it fail loudly.
TensorBuffer* alloc_virtual(int32_t dtype, const size_t* shape, int ndim);
void release(TensorBuffer* t);
void retain(TensorBuffer* t);
// Scratch device memory from the same pool, released with pool_free.
void* pool_alloc(size_t bytes, size_t* bucket_out);
void pool_free(void* p, size_t bucket);
// HIP graph capture: buffers handed out between pool_capture_begin(g) and
// pool_capture_end(g) stay reserved for graph g (never reused by others)
// until pool_release_graph(g).
void pool_capture_begin(int graph);
void pool_capture_end(int graph);
void pool_release_graph(int graph);

// Host -> device copy on the runtime stream via pinned staging.
void upload(void* dst, const void* src, size_t bytes);
// Device -> host copy after waiting for the producing work.
void download(void* dst, const TensorBuffer* t, size_t bytes);
// Fill the tiles a causal attention forward left unwritten
// (Storage::upper_unwritten_t) before anything other than the fused
// backward reads the tensor; no-op otherwise.
void materialize_upper_tiles(TensorBuffer* t);

// Device-side error flag (index out of range in gathers); checked at flush.
int32_t* device_error_flag();

// ---- RNG (metal.rs:1690-1759) ----------------------------------------------
void philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
uint64_t rng_next_call();

// ---- kernel launch wrappers (k_*.hip) --------------------------------------
namespace k {
// k_rng.hip: Philox4x32-10 on the device (the host generator's words).
// randn: Box-Muller of pair k (counter [k, 0, 0, 0], key = call) in f64.
void randn(float* out, size_t n, uint64_t call, hipStream_t s);
// rand_tokens: x[i] = rand_int(vocab) with call index cx + i, y[i] with cy + i
// (vocab >= 1); `calls` (device, 2 words), when given, supplies cx and cy.
void rand_tokens(int32_t* x, int32_t* y, size_t n, const uint64_t* calls, uint64_t cx, uint64_t cy, uint32_t vocab,
                 hipStream_t s);
// batch_windows: B sequences of T tokens at starts rand_int(range) drawn with
// call indices call0 .. call0 + B - 1; y is x shifted by one token.
void batch_windows(const int32_t* data, int32_t* x, int32_t* y, size_t B, size_t T, uint64_t call0, uint64_t range,
                   int32_t* starts, hipStream_t s);
enum BinOp : int { ADD = 0, SUB = 1, MUL = 2, DIV = 3 };
enum UnOp : int { RELU = 0, SIGMOID, TANH, EXP, LOG, SQRT, ABS, GELU, NEG_UNUSED };
enum UnBwd : int { B_SIGMOID = 0, B_RELU, B_TANH, B_SQRT, B_ABS, B_GELU, B_EXP, B_LOG };

struct BcastDesc {          // NumPy right-aligned broadcast of (p op q) into out
  int ndim;
  uint32_t out_shape[kMaxRank];
  uint32_t p_stride[kMaxRank];  // 0 where p is broadcast
  uint32_t q_stride[kMaxRank];
};

// out[i] = p[i] op q[i]
void binary_same(int op, const float* p, const float* q, float* out, size_t n, hipStream_t s);
// out = p op q with q broadcast along rows: q_flat = i % qn (trailing-block broadcast)
void binary_rowbcast(int op, const float* p, const float* q, float* out, size_t n, size_t qn, hipStream_t s);
// out = p op q with p broadcast: p_flat = i % pn
void binary_rowbcast_rev(int op, const float* p, size_t pn, const float* q, float* out, size_t n, hipStream_t s);
// out = p op q[0] (qdev != null: scalar read from device) or p op qval
void binary_scalar(int op, const float* p, const float* qdev, float qval, bool scalar_on_right,
                   float* out, size_t n, hipStream_t s);
void binary_general(int op, const float* p, const float* q, float* out, size_t n, const BcastDesc& d, hipStream_t s);
void unary(int op, const float* x, float* out, size_t n, hipStream_t s);
void unary_bwd(int op, const float* xy, const float* dout, float* out, size_t n, hipStream_t s);
// out = x converted f32 -> bf16 (to_bf16, round to nearest even) or bf16 -> f32 (exact).
void convert_f32_bf16(const void* x, void* out, size_t n, bool to_bf16, hipStream_t s);
// Many f32 -> bf16 conversions (round to nearest even) in one launch.
struct Bf16Copy {
  const float* src;
  void* dst;
  size_t n;
};
void to_bf16_multi(const Bf16Copy* segs_host, int count, hipStream_t s);
// Many split copies in one launch: dst (bf16) gets the h, m and l pieces of
// src's n values as three planes of n (the pieces the split GEMM forms).
void to_split3_multi(const Bf16Copy* segs_host, int count, hipStream_t s);
void fill(float* out, float v, size_t n, hipStream_t s);
void fill_bytes0(void* out, size_t bytes, hipStream_t s);
void fill_from_device(float* out, const float* v, size_t n, hipStream_t s);
void eq(const float* a, const float* b, float* out, size_t n, hipStream_t s);
void rsqrt_eps(const float* v, float eps, float* out, size_t n, hipStream_t s);
void copy(const void* src, void* dst, size_t bytes, hipStream_t s);
void causal_mask(float* out, size_t t, hipStream_t s);
void iota_rows(int32_t* out, size_t rows, size_t t, hipStream_t s);

// Axis reductions over a contiguous [outer, axis, inner] view.
enum RedOp : int { R_SUM = 0, R_MEAN = 1, R_MAX = 2, R_VAR = 3 };
void reduce_axis(int op, const float* x, float* out, size_t outer, size_t axis, size_t inner, hipStream_t s);
// reduce_axis with its temporaries (split partials; the variance's mean) in
// a caller's device buffer of `scratch_floats` floats instead of the pool;
// the same plan and kernels, so the same values.  reduce_axis_scratch_floats
// is the size that call needs (0: none).
size_t reduce_axis_scratch_floats(int op, const float* x, const float* out, size_t outer, size_t axis, size_t inner);
void reduce_axis_scratch(int op, const float* x, float* out, size_t outer, size_t axis, size_t inner, float* scratch,
                         size_t scratch_floats, hipStream_t s);
// P = softmax over the last axis of (S * scale[0]) + mask[row % mask_rows],
// each op rounded as the separate broadcast kernels round it.
void scale_mask_softmax(const float* S, const float* scale, const float* mask, float* P, size_t rows, size_t axis,
                        size_t mask_rows, hipStream_t s);
// P = softmax(Q K^T * scale[0] + mask) over each query row of every head,
// Q, K: [bh, t, hs], mask: [t, t], P: [bh, t, t]; the same values as
// gemm(Q, K^T) followed by scale_mask_softmax.  causal: the mask is
// -1e9 above the diagonal and 0 elsewhere (key tiles wholly above a row
// block are skipped, and the mask is applied arithmetically: mask may be
// null).  Returns false (nothing launched) for shapes the kernel is not
// built for.
bool attn_scores_supported(size_t bh, size_t t, size_t hs);
bool attn_scores_softmax(const float* Q, const float* K, const float* scale, const float* mask, float* P, size_t bh,
                         size_t t, size_t hs, bool causal, hipStream_t s);
// dS = softmax_bwd(P, dO @ V^T) * scale[0] per head (P, dS: [bh, t, t];
// V: [bh, t, hs]); dO of head b is read at dO + (b / heads) * t * ldo +
// (b % heads) * hs with row stride ldo (ldo = hs, heads = 1: dense
// [bh, t, hs]).  Same values as gemm + softmax_bwd + the scalar multiply.
bool attn_scores_bwd(const float* dO, size_t ldo, size_t heads, const float* V, const float* P, const float* scale,
                     float* dS, size_t bh, size_t t, size_t hs, bool causal, hipStream_t s);
// attn_scores_softmax, and with O non-null also O = P @ V (V [bh, t, hs])
// from the same kernel: head b's row i, column d at O + (b / heads) * t * ldo
// + (b % heads) * hs + i * ldo + d.  Same values as gemm(P, V).
// causal && !full: the 32 x 32 tiles of P wholly above the diagonal are
// not written (no reader of this P looks at them).
bool attn_fwd(const float* Q, const float* K, const float* V, const float* scale, const float* mask, float* P, float* O,
              size_t ldo, size_t heads, size_t bh, size_t t, size_t hs, bool causal, hipStream_t s, bool full = true);
// The zero tiles attn_fwd(full = false) left unwritten: P [bh, t, t].
void attn_zero_upper_tiles(float* P, size_t bh, size_t t, hipStream_t s);
// attn_scores_bwd, and with dQ non-null also dQ = Dq + dS @ K (K, dQ, Dq
// dense [bh, t, hs]; Dq may be null) from the same kernel.  Same values as
// gemm(dS, K) with the addend.
// With kv non-null (needs dQ) the same kernel also forms, per head,
// dK = Dk + dS^T @ Q and dV = Dv + P^T @ dO (Q, dK, dV, Dk, Dv dense
// [bh, t, hs]; the addends may be null): the same values as the two GEMMs.
struct AttnKV {
  const float* Q;
  float* dK;
  const float* Dk;
  float* dV;
  const float* Dv;
};
// causal && !full: dS's tiles wholly above the diagonal are not written (a
// scratch dS that only this kernel reads).
bool attn_bwd(const float* dO, size_t ldo, size_t heads, const float* V, const float* P, const float* scale, float* dS,
              const float* K, float* dQ, const float* Dq, size_t bh, size_t t, size_t hs, bool causal, hipStream_t s,
              const AttnKV* kv = nullptr, bool full = true);
// Flash attention (online softmax, no [bh, t, t] buffers): t any multiple
// of 32, hs 32 or 64.  Forward: O = softmax(Q K^T * scale[0] (+ causal
// mask)) @ V written at O + (b / heads) * t * ldo + (b % heads) * hs +
// i * ldo (ldo = heads * hs: the [B*T, C] layout; ldo = hs, heads = 1:
// dense), and lse[b * t + i] = row max + log(row sum).  bf16: products on
// the bf16 MFMA (autocast).  qkv_bf16 (with bf16): Q, K, V stored in bf16,
// and in flash_bwd dQ, dK, dV written in bf16 (no addends).  False (nothing
// launched) when the shape or an alignment does not fit.
bool flash_supported(size_t bh, size_t t, size_t hs);
bool flash_fwd(const float* Q, const float* K, const float* V, const float* scale, float* O, size_t ldo, size_t heads,
               float* lse, size_t bh, size_t t, size_t hs, bool causal, bool bf16, hipStream_t s,
               bool qkv_bf16 = false);
// Backward: dQ = Dq + dS K, dK = Dk + dS^T Q, dV = Dv + P^T dO with P
// recomputed from lse and dS = P (dP - rowsum(dO O)) scale; O and dO use the
// forward's O addressing, Q K V dQ dK dV (and the optional addends) are
// dense [bh, t, hs]; dsum is [bh, t] scratch.
struct FlashBwd {
  const float *Q, *K, *V, *O, *dO, *lse, *scale;
  float *dQ, *dK, *dV, *dsum;
  const float *Dq, *Dk, *Dv;
};
bool flash_bwd(const FlashBwd& a, size_t ldo, size_t heads, size_t bh, size_t t, size_t hs, bool causal, bool bf16,
               hipStream_t s, bool qkv_bf16 = false);
// The autocast scope's state (GEMMs and flash attention on the bf16 MFMA).
bool autocast_on();
// Whether f32 GEMMs (and the fused attention kernels, which reproduce the
// composed GEMMs' bits) compute their products as split bf16 pieces
// (malus_gemm_set_f32_split; k_split.h).
bool gemm_f32_split();
// Sum over the axis of x * y (y has x's layout); each product rounded to f32.
void reduce_axis_prod(const float* x, const float* y, float* out, size_t outer, size_t axis, size_t inner, hipStream_t s);
// The split of reduce_axis_prod's column reduction over [axis, inner]
// (outer = 1): nsplit chunks of `chunk` rows, row_threads rows interleaved
// per chunk.  False when it does not split on the float4 path or walks
// contiguous runs of rows instead.
bool col_prod_split(size_t axis, size_t inner, uint32_t* nsplit, size_t* chunk, int* row_threads);
// out[c] = the sum over s of partial[s * cols + c], as that reduction combines them.
void col_combine_sum(const float* partial, float* out, size_t cols, uint32_t nsplit, size_t axis, hipStream_t s);
// col_combine_sum of a pool block the call takes over (pool_free'd after its
// last use).  defer (and nsplit % 4 == 0): the sum is queued, and runs with
// every other queued one in one launch at the thread's next
// col_combine_flush; `out` must not be read before then.
void col_combine_sum_owned(float* partial, size_t bucket, float* out, size_t cols, uint32_t nsplit, size_t axis,
                           bool defer, hipStream_t s);
void col_combine_flush(hipStream_t s);
// Broadcast [outer, inner] back to [outer, axis, inner] (expand_axis).
void expand_axis(const float* small, float* out, size_t outer, size_t axis, size_t inner, hipStream_t s);

// Row ops over [outer, axis, inner] (inner may be > 1).
void softmax(const float* x, float* out, size_t outer, size_t axis, size_t inner, hipStream_t s);
void softmax_bwd(const float* y, const float* dout, float* out, size_t outer, size_t axis, size_t inner, hipStream_t s);
// With w (last axis only): also out = y * w broadcast over rows.
// out_bf16: out (the affine output) stored in bf16, rounded to nearest even.
void layernorm(const float* x, float* y, float* var, size_t outer, size_t axis, size_t inner, float eps, hipStream_t s,
               const float* w = nullptr, float* out = nullptr, bool out_bf16 = false);
// With addend: dx = addend + VJP (gradient accumulation folded in).  With w
// (last axis only): dout is the gradient of y * w, and dy = dout * w is formed
// in the kernel.
// layernorm_bwd with the scale w, plus dw = reduce_axis_prod(dout, y) over
// the rows, from one row kernel and the combine (bit-identical to the two
// separate calls).  False (nothing launched) when the shape has no such form.
// defer_dw: dw's combine is queued for col_combine_flush.
bool layernorm_bwd_scale(const float* y, const float* var, const float* dout, float* dx, float* dw, size_t rows,
                         size_t axis, float eps, hipStream_t s, const float* addend, const float* w,
                         bool defer_dw = false);
void layernorm_bwd(const float* y, const float* var, const float* dout, float* dx, size_t outer, size_t axis, size_t inner,
                   float eps, hipStream_t s,
                   const float* addend = nullptr, const float* w = nullptr);
// probs = softmax(logits) rows; nll[i] = -log(probs[i, t_i]).
void ce_fwd(const float* logits, const int32_t* tgt, float* probs, float* nll, size_t n, size_t v, int32_t* err, hipStream_t s);
// scale = dout[0] / n when dout is given (read on the device), else scale_host.
void ce_bwd(const float* probs, const int32_t* tgt, const float* dout, float scale_host, float* dx, size_t n, size_t v,
            hipStream_t s);
// nll[i] = -log(probs[i, t_i])  (cross_entropy.ml:13-16)
void nll_gather(const float* probs, const int32_t* tgt, float* nll, size_t n, size_t v, int32_t* err, hipStream_t s);

// Gathers / index ops.
void embedding(const float* w, const int32_t* idx, float* out, size_t t, size_t v, size_t d, int32_t* err, hipStream_t s);
// out = embedding(wa, ia) + embedding(wb, ib) in one pass (d % 4 == 0;
// 16-byte aligned tables and output).
void embedding2(const float* wa, const int32_t* ia, size_t va, const float* wb, const int32_t* ib, size_t vb, float* out,
                size_t t, size_t d, int32_t* err, hipStream_t s);
void embedding_bwd(const float* dout, const int32_t* idx, float* dw, size_t t, size_t v, size_t d, hipStream_t s);
// embedding_bwd of two tables (va and vb rows of width d) indexed by idx_a
// and idx_b (t each) with one dout, from one list launch and one sum launch
// (the same values as two embedding_bwd calls).  False (nothing launched)
// when the shapes do not take that form.
bool embedding_bwd2(const float* dout, const int32_t* idx_a, float* dw_a, size_t va, const int32_t* idx_b,
                    float* dw_b, size_t vb, size_t t, size_t d, hipStream_t s);
void permute(const float* x, float* out, int ndim, const size_t* in_shape, const size_t* perm, hipStream_t s);

// Operand addressing for gemm_mapped: element (i, j) of a stored matrix
// (rows i, columns j) of batch b sits at  b-map(b) + r-map(i) + c-map(j)
// elements (floats, or bf16 for an operand GemmLayouts::io marks) past the
// operand's pointer, each map being
//   x -> (x / div) * s1 + (x % div) * s0     (div == 0: x * s0),
// which covers dense row-major storage ({0, 0, ld} rows, {0, 0, 1} columns)
// and the head-folded views of multi-head attention (a [B*T, H*hs] matrix
// stored as [B, H, T, hs], or per-head [T, hs] matrices inside [B, T, H, hs]).
// Offsets stay below 2^29 floats (2^31 bytes), so the fields are 32-bit.
struct GemmMap { int div, s1, s0; };
struct GemmLayout { GemmMap b, r, c; };
// ext_a / ext_b: elements addressable past A / B (the whole allocation).
// tri_a: every stored A matrix is square and lower-triangular, with exact
// zeros above the diagonal (causal attention probabilities and their
// gradients); a tile then skips the k slabs whose A values are all zero,
// which leaves every sum's value unchanged.
// ngroup > 1 (gemm_grouped): up to 3 products with this one shape and
// layout, group g reading ga[g] / gb[g] and writing gc[g].
// io: operands stored in bf16 (kIo* bits; such a GEMM runs on the bf16 MFMA
// whatever the autocast state, and its maps and ext_* count bf16 elements).
constexpr int kIoA16 = 1;  // A stored in bf16
constexpr int kIoB16 = 2;  // B stored in bf16
constexpr int kIoC16 = 4;  // C written in bf16 (no addend, no K split)
constexpr int kIoE16 = 8;  // the GELU epilogues' E (written or read) in bf16
constexpr int kIoB3 = 16;  // B as the three bf16 planes of its split pieces (split products only;
                           // plane p of element x at x + p * ext_b)
struct GemmLayouts {
  GemmLayout a, b, c;
  int ext_a, ext_b;
  int tri_a = 0;
  int ngroup = 1;
  int io = 0;
  const float* ga[3] = {nullptr, nullptr, nullptr};
  const float* gb[3] = {nullptr, nullptr, nullptr};
  float* gc[3] = {nullptr, nullptr, nullptr};
};
inline GemmLayout dense_layout(long ld, long batch_stride) {
  return {{0, 0, (int)batch_stride}, {0, 0, (int)ld}, {0, 0, 1}};
}

// Batched GEMM: C[b] = op(A[b]) @ op(B[b]); transA: A stored [K,M]; transB: B stored [N,K].
// strideA/B/C are element strides between batches (0 broadcasts).
// With D (C's layout and batch stride), C = D + op(A) @ op(B): the GEMM
// result is rounded to f32 before the add, exactly as a separate add of the
// stored product would round.
// io: kIoA16 / kIoB16 operands stored in bf16 (LDS-DMA shapes only; fails
// loudly otherwise).
void gemm(const float* A, const float* B, float* C, int batch, int M, int N, int K, bool transA, bool transB,
          long strideA, long strideB, long strideC, hipStream_t s, const float* D = nullptr, int io = 0);
// gemm with every operand addressed through its layout (D shares C's).
// Returns false, launching nothing, when the LDS-DMA kernels cannot take
// the layouts: K % 16 != 0, a contiguous dimension whose maps are not unit
// stride in runs of 4, a k map whose div is not a multiple of 16, a C row
// map whose div is not a multiple of 32, or offsets of 2^31 bytes or more.
// GEMMs with a fused GELU (dense, batch 1, LDS-DMA path; false, launching
// nothing, when the shape does not fit it):
//   forward  (backward = false): C = A @ B and E = gelu(C);
//   backward (backward = true, transB): C = gelu_bwd(E, A @ B^T) (+ D), with E
//   the GELU's input: the GELU VJP of the product, rounded as the separate
//   kernels round it.
// io: kIoA16 for a bf16 A; kIoE16 for a bf16 E (the forward's gelu(C)
// output, the backward's GELU input); kIoC16 for a bf16 C (backward, no D).
bool gemm_gelu(const float* A, const float* B, float* C, float* E, int M, int N, int K, bool transB, bool backward,
               hipStream_t s, const float* D = nullptr, int io = 0);
// Grouped GEMMs on the mapped LDS-DMA kernel (batch 1): L.ngroup products
// of one shape and layout, operands L.ga / L.gb.
//   accumulate = false: L.gc[g] = op(A_g) @ op(B_g), all groups in one
//     launch (split-K as for a single product of the shape);
//   accumulate = true: C = ((D + op(A_0) @ op(B_0)) + op(A_1) @ op(B_1)) + ...,
//     each product rounded to f32 before its add, as one GEMM per group with
//     chained addends would round (no split).
// Returns false, launching nothing, where gemm_mapped would.
bool gemm_grouped(int M, int N, int K, bool transA, bool transB, const GemmLayouts& L, float* C, bool accumulate,
                  hipStream_t s, const float* D = nullptr, double* flops = nullptr);
// flops (optional): the multiply-add work launched (less than 2 M N K when
// tri_a skips zero slabs).
bool gemm_mapped(const float* A, const float* B, float* C, int batch, int M, int N, int K, bool transA, bool transB,
                 const GemmLayouts& L, hipStream_t s, const float* D = nullptr, double* flops = nullptr);

// Fused Adam + L2 update (examples/nanogpt_modular.ml:97-108 op order).
// One parameter tensor of a multi-tensor Adam update (device pointers).
struct AdamSeg {
  const float *p, *g, *m, *v;
  float *po, *mo, *vo;
  size_t n;
};
constexpr size_t kAdamChunk = 1024;  // floats per workgroup
// Every tensor of `segs` in one launch; same per-element expression as adam_l2.
void adam_l2_multi(const AdamSeg* segs_host, int count, float lr, float b1, float b2, float omb1, float omb2, float bc1,
                   float bc2, float eps, float wd, hipStream_t s, const float* bc_dev = nullptr);
void adam_l2(const float* p, const float* g, const float* m, const float* v, float* p_out, float* m_out, float* v_out,
             size_t n, float lr, float b1, float b2, float omb1, float omb2, float bc1, float bc2, float eps, float wd,
             hipStream_t s);
}  // namespace k

// ---- per-kernel timing (bench instrumentation) ------------------------------
struct KTimer;
KTimer* ktimer_begin(const char* cls);     // null when timing is off
void ktimer_end(KTimer* t, double algorithmic_units);

}  // namespace malus
