/*
 * libmalus_hip — the malus runtime C ABI on AMD MI355X (gfx950).
 *
 * Drop-in for crates/malus-runtime (the Metal runtime): every symbol the
 * Cranelift JIT imports through RuntimeSymbols
 * (crates/malus-codegen-cpu/src/lib.rs:115-184) plus the Rust-side helpers
 * of crates/malus-runtime/src/lib.rs:117-176, with the same names, argument
 * meaning and ownership rules.  Each declaration cites the reference
 * function it replaces.
 *
 * Handles: an int64_t tensor handle is an opaque pointer; 0 is "null".
 * Returned handles carry refcount 1 and are owned by the caller; input
 * handles are borrowed.  Errors follow the reference's panic model
 * ("malus: ..." on stderr, then abort) unless malus_set_abort_on_error(0)
 * selects return mode (the call returns 0 and malus_last_error() holds the
 * message).
 *
 * Execution: every GPU op is enqueued on one in-order HIP stream; a host
 * read (tensor_print, malus_tensor_get_f32, malus_tensor_read) waits only
 * when the tensor still has an unfinished write.
 */
#ifndef MALUS_HIP_H
#define MALUS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype tags (metal.rs:26-50): F32=0 F16=1 BF16=2 I8=3 I16=4 I32=5 I64=6
 * U8=7 U16=8 U32=9 U64=10; tensors support F32, I32 and I64. */

/* ---- context ---------------------------------------------------------- */
/* Initialize the device context (lazy in every entry point; explicit here).
 * Replaces the lazy MetalContext singleton, metal.rs:62-112. */
void malus_init(void);
/* runtime_init(&HashMap<u64, String>) as a C ABI, metal.rs:304-336.
 * Builtin stdlib kernels are recognized by a "//@malus-builtin <name>" tag;
 * other sources are HIP C++ compiled with hipRTC (cached by source text). */
void malus_runtime_init(const uint64_t* ids, const char* const* sources, size_t n);
int malus_kernel_is_builtin(uint64_t id);
/* No reference counterpart: compile HIP source for `arch` with the options
 * malus_runtime_init uses for user kernels (no device needed).  Returns the
 * code object size, 0 on failure (compiler log in `log`); copies the object
 * into `code` when `cap` is large enough. */
size_t malus_rtc_compile(const char* src, const char* arch, void* code, size_t cap, char* log, size_t log_cap);

/* ---- allocation-free reduction ------------------------------------------ */
/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The values of malus_std_reduce_fwd(op, x, axis, keepdim)
 * (op: 0 sum, 1 mean, 2 max, 3 population variance) for a contiguous f32
 * tensor of `shape` at device address `x`, written to the caller's device
 * buffer `out` (outer * inner floats; keepdim only changes the shape), with
 * the same kernels and plan.  Its split partials and the variance's mean
 * live in a fixed 4 MiB device array of the library (one per GPU, held until
 * the process ends, set up by malus_init); a reduction needing more is
 * rejected with an error.  No hipMalloc/hipFree is called.  The work is
 * enqueued on the library's stream (gpu_barrier() waits for it); calls on one
 * GPU share the array, so calls that overlap (several host threads) race.
 * With 16-byte-aligned x and out the values equal malus_std_reduce_fwd's.
 * Returns 0, or -1 in return-error mode. */
int malus_std_reduce_noalloc(int32_t op, const float* x, const size_t* shape, size_t ndim, int64_t axis, float* out);

/* ---- HIP emitter (crates/malus-codegen-gpu/src/lib.rs) -------------------- */
/* compile_kernels (codegen-gpu/lib.rs:95-155) as a C ABI.  `program` is malus
 * source; each top-level `kernel` item is parsed, type-checked with the
 * reference sema's kernel-body rules and lowered to HIP C++ for hipRTC
 * (implicit-map bodies to the v1 ABI, lib.rs:432-562; explicit bodies to the
 * v2 ABI, lib.rs:564-1006); other items are skipped.  `builtins` names the
 * synthesized kernels the program's fn bodies use ("malus_add" ...
 * "malus_rdiv_scalar", "relu" ... "abs"; lib.rs:373-418), which sema collects
 * from typed fn bodies.  Ids are process-global and increase in the
 * reference's order: user kernels, tensor-tensor, scalar-broadcast, unary.
 * flags bit 0: prefix the sources of kernels the runtime implements by hand
 * (the stdlib kernels and builtins) with "//@malus-builtin <name>", so
 * malus_runtime_init binds the hand-written kernel.  Returns NULL on error
 * (malus_last_error() in return mode). */
typedef struct malus_registry malus_registry;
malus_registry* malus_compile_kernels(const char* program, const char* const* builtins, size_t nbuiltins, int flags);
size_t malus_registry_len(const malus_registry* r);
uint64_t malus_registry_id(const malus_registry* r, size_t i);
const char* malus_registry_name(const malus_registry* r, size_t i);
const char* malus_registry_source(const malus_registry* r, size_t i);
int malus_registry_lookup(const malus_registry* r, const char* name, uint64_t* id);
void malus_registry_free(malus_registry* r);

/* ---- tensor creation and lifetime (metal.rs:340-558) -------------------- */
int64_t tensor_alloc_gpu(int32_t dtype, const size_t* shape, size_t ndim, const void* data); /* metal.rs:341-348 */
int64_t tensor_alloc_zeros_gpu(const size_t* shape, size_t ndim);                          /* metal.rs:458-484 */
int64_t tensor_alloc_ones_gpu(const size_t* shape, size_t ndim);                           /* metal.rs:486-492 */
void tensor_retain(int64_t h);                                                              /* metal.rs:499-507 */
void tensor_release(int64_t h);                                                             /* metal.rs:520-552 */
void tensor_free(int64_t h);                                                                /* metal.rs:556-558 */

/* ---- metadata and host reads (metal.rs:560-672, 1763-1769) -------------- */
void tensor_print(int64_t h);                     /* metal.rs:561-588 (Rust `{}` float formatting) */
int64_t tensor_len(int64_t h);                    /* metal.rs:651-655 */
int64_t tensor_ndim(int64_t h);                   /* metal.rs:657-661 */
int64_t tensor_dim(int64_t h, int64_t i);         /* metal.rs:663-672 (negative i allowed) */
float malus_tensor_get_f32(int64_t h, int64_t i); /* metal.rs:1763-1769 */
/* No reference counterpart: bulk host I/O used by tests and the bench. */
int32_t malus_tensor_dtype(int64_t h);
void malus_tensor_shape(int64_t h, size_t* out /* [8] */);
void malus_tensor_read(int64_t h, void* dst, size_t bytes);
void malus_tensor_write(int64_t h, const void* src, size_t bytes);
/* The device address of a tensor's storage; NULL for a shape-only handle.
 * Writes made through it are not tracked by tensor_is_pending. */
void* malus_tensor_device_ptr(int64_t h);
size_t malus_format_f32(float v, char* buf, size_t cap);

/* ---- synchronization (metal.rs:201-259, 677-694) ------------------------ */
void gpu_barrier(void);                 /* metal.rs:677-694 */
void malus_flush_if_pending(int64_t h); /* flush_if_pending, metal.rs:244-252 */
int tensor_is_pending(int64_t h);       /* metal.rs:256-259 */

/* ---- kernel launches (metal.rs:1860-2065) -------------------------------- */
int64_t kernel_dispatch(uint64_t kernel_id, const int64_t* handles, size_t count); /* metal.rs:1860-1931 */
int64_t kernel_dispatch_v2(uint64_t kernel_id, const int64_t* handles, size_t handle_count,
                           const size_t* grid_dims /*[3]*/, const size_t* tg_dims /*[3]*/,
                           const size_t* out_shape, size_t out_ndim, int32_t out_dtype_tag,
                           const void* uniforms, size_t uniforms_bytes); /* metal.rs:1944-2065 */

/* ---- matmul, shapes, masks, RNG ----------------------------------------- */
int64_t tensor_matmul(int64_t a, int64_t b); /* metal.rs:820-962 (split bf16 products or FP32 MFMA: malus_gemm_set_f32_split) */
int64_t tensor_reshape(int64_t h, const size_t* dims, size_t ndim);     /* metal.rs:1421-1435 */
int64_t tensor_permute(int64_t h, const size_t* perm, size_t ndims);    /* metal.rs:1405-1417 */
int64_t tensor_causal_mask(int64_t t);                                  /* metal.rs:1600-1612 */
int64_t tensor_randn(const size_t* shape, size_t ndim);                 /* metal.rs:1720-1740 */
float malus_rand_uniform(void);                                         /* metal.rs:1744-1750 */
int64_t malus_rand_int(int64_t n);                                      /* metal.rs:1752-1759 */
/* No reference counterpart: read/set the per-thread RNG call counter. */
/* No reference counterpart: the device-side data path.  randn with the
 * stream of tensor_randn (metal.rs:1720-1740: the same Philox words and the
 * same f64 Box-Muller), generated on the device.  batch_windows builds the
 * nanogpt_modular.ml:170-177 batch from a device-resident 1-D i32 token
 * stream: B sequence starts rand_int(len - T - 1) (B RNG calls, as the host
 * loop makes them) and x/y windows of T tokens (y shifted by one), as new
 * [B*T] i32 tensors; starts_out (host int32[B], optional) gets the starts. */
int64_t malus_randn_device(const size_t* shape, size_t ndim);
void malus_batch_windows(int64_t data, int64_t B, int64_t T, int64_t* x_out, int64_t* y_out, int32_t* starts_out);
/* No reference counterpart (device-side data path): n i.i.d. token ids,
 * out[i] = rand_int(vocab) with call index call + i, the ids of the host
 * builtin's loop (metal.rs:1752-1759), drawn on the device; a new [n] i32. */
int64_t malus_rand_tokens_device(uint64_t call, size_t n, int64_t vocab);
uint64_t malus_rng_get_counter(void);
void malus_rng_set_counter(uint64_t v);

/* ---- Buffer<i32> staging (buffer.rs:1-50) -------------------------------- */
int64_t malus_buffer_i32(int64_t len);
int64_t malus_buffer_get_i32(int64_t h, int64_t i);
void malus_buffer_set_i32(int64_t h, int64_t i, int64_t v);
void malus_buffer_free(int64_t h);
int64_t malus_buffer_freeze_i32(int64_t h);

/* ---- autograd tape (tape.rs) -------------------------------------------- */
void tape_record_binop(int32_t op_tag, int64_t a, int64_t b, int64_t out);                    /* tape.rs:206-218 */
void tape_record_unary(int32_t op_tag, int64_t x, int64_t out);                               /* tape.rs:221-231 */
void tape_record_reduce(int32_t op_tag, int64_t x, int64_t out, int64_t axis, int64_t keepdim); /* tape.rs:236-255 */
void tape_record_perm(int32_t op_tag, int64_t x, int64_t out, const size_t* dims, size_t ndims); /* tape.rs:259-283 */
void tape_record_layernorm(int32_t op_tag, int64_t x, int64_t out, int64_t var_h, int64_t axis); /* tape.rs:289-310 */
void tape_record_cross_entropy(int32_t op_tag, int64_t logits, int64_t out, int64_t softmax_h,
                               int64_t targets);                                               /* tape.rs:315-337 */
void tape_record_embedding(int32_t op_tag, int64_t weight, int64_t indices, int64_t out);      /* tape.rs:342-353 */
void tape_register_leaf(int64_t h);                                                            /* tape.rs:358-363 */
void tape_pause(void);                                                                         /* tape.rs:365-368 */
void tape_resume(void);                                                                        /* tape.rs:370-373 */
void tape_clear(void);                                                                         /* tape.rs:377-389 */
int64_t tape_get_grad(int64_t h);                                                              /* tape.rs:395-411 */
void backward(int64_t loss);                                                                   /* tape.rs:421-729 */
void tape_zero_grad(const int64_t* handles, size_t count);                                     /* tape.rs:757-774 */
void tape_reset(void);                                                                         /* tape.rs:735-750 */
void tape_register_backward_fn(int32_t slot, size_t fnptr);                                    /* tape.rs:143-147 */
/* 1 (default): gradient accumulation folded into matmul/layernorm VJP kernels; 0: separate adds (same values). */
void malus_tape_set_fused_vjps(int on);
/* No reference counterpart: the pointer currently held by a BwdSlot. */
size_t malus_tape_backward_fn(int32_t slot);
size_t malus_tape_len(void);
void malus_tape_registry_lens(size_t* out2);

/* ---- bench timer (bench.rs:1-76) ----------------------------------------- */
void bench_enable(void);
void bench_reset(void);
void bench_step_begin(void);
void bench_step_end(void);
/* bench_report (bench.rs:51-70) through out-params; returns 0 when <= 3 steps. */
int bench_report(double* median_ms, double* min_ms, double* max_ms, int64_t* warm_steps);
void malus_bench_record(double ms);

/* ---- counters and pool (runtime/lib.rs:1-94, metal.rs:114-199) ----------- */
int64_t malus_cpu_compute_count(void); /* always 0: the library has no CPU compute path */
void malus_cpu_compute_reset(void);
void malus_rc_counts(int64_t* out3 /* retain, release, alloc */);
void malus_rc_reset(void);
void malus_record_diff(float v);
float malus_gradcheck_max_diff(void);
void malus_gradcheck_reset(void);
void malus_pool_stats(int64_t* out4 /* hits, misses, pooled_bytes, peak_device_bytes */);
int64_t malus_pool_live_bytes(void);
size_t malus_pool_buckets(size_t* sizes, size_t* counts, size_t cap);
void malus_pool_reset(void);
void malus_set_mem_budget(int64_t bytes);
/* Fault injection for tests of error paths (no reference counterpart): the
 * pool allocation after the next n fails with a malus error, once; n < 0
 * turns it off.  The failure is raised on the host before the buffer's
 * first use, so no kernel sees it. */
void malus_fail_alloc_after(int64_t n);
size_t malus_alloc_histogram(size_t* sizes, uint64_t* counts, size_t cap);

/* ---- instrumentation and errors (no reference counterparts) ------------- */
void malus_ktimer_enable(int on);
/* Tuning: pin the GEMM block tile to (64*tm) x (64*tn); (0, 0) = automatic. */
int malus_gemm_set_tile(int tm, int tn);
/* Tuning: workgroups a split-K GEMM aims for; 0 = the cost model decides. */
void malus_gemm_set_split(int target_blocks);
/* Tuning: 0 keeps every GEMM on the register-staged path; 1 (default) allows the LDS-DMA path. */
void malus_gemm_set_dma(int on);
/* f32 GEMM arithmetic (no reference counterpart; the products of
 * metal.rs:802-962): 1 (default) computes every f32 GEMM on the LDS-DMA
 * kernels, and the fused attention kernels' products, as the sum of six
 * exact bf16 piece products on the bf16 MFMA (each operand value split
 * exactly into three bf16 pieces, f32 accumulation); 0 runs them on the
 * FP32 MFMA.  The environment variable MALUS_F32_GEMM=fp32 sets 0 at
 * start-up.  Returns the previous setting.  A captured graph keeps the
 * arithmetic it was captured with. */
int malus_gemm_set_f32_split(int on);
/* The `with autocast:` scope of docs/adr/0037-bf16-autocast.md:5-12 (the
 * reference fixes the policy, not yet an entry point): while on, every GEMM
 * (tensor_matmul, the model's projections and their VJPs) rounds its f32
 * operands to bf16 (nearest even) and accumulates in f32 on the bf16 MFMA;
 * tensors, parameters, gradients, optimizer state, reductions and the fused
 * attention stay f32.  Returns the previous state, which the scope's exit
 * passes back.  A captured step keeps the precision it was captured with. */
int malus_autocast(int on);
/* Fused attention scores softmax(q @ k^T * scale + mask, axis=2) for q, k
 * [bh, t, hs] (t, hs in {256,64}, {128,64}, {64,32}, {64,64}); the kernel the
 * model's fused forward uses for nanogpt_modular.ml:57-61.  causal != 0
 * promises the -1e9-above-the-diagonal mask of tensor_causal_mask. */
int64_t malus_std_attn_scores_softmax(int64_t q, int64_t k, int64_t scale, int64_t mask, int32_t causal);
/* Its VJP fused with the score products' gradient input:
 * softmax_bwd(p, dout @ v^T, axis=2) * scale for dout, v [bh, t, hs], p [bh, t, t]
 * (the kernel the fused attention backward uses; transformer_bwd.ml:15-20 then the
 * scale multiply's VJP). */
int64_t malus_std_attn_scores_bwd(int64_t dout, int64_t v, int64_t p, int64_t scale, int32_t causal);
/* The whole fused attention forward: returns attn @ v [bh, t, hs] for
 * attn = malus_std_attn_scores_softmax(q, k, scale, mask, causal), written
 * with attn from one kernel (nanogpt_modular.ml:57-62); *p_out (if non-null)
 * receives attn. */
int64_t malus_std_attn_fwd(int64_t q, int64_t k, int64_t v, int64_t scale, int64_t mask, int32_t causal,
                           int64_t* p_out);
/* malus_std_attn_scores_bwd, and dq = ds @ k [bh, t, hs] (the scores
 * product's VJP for q) from the same kernel into *dq_out (if non-null). */
int64_t malus_std_attn_bwd(int64_t dout, int64_t v, int64_t p, int64_t scale, int64_t k, int32_t causal,
                           int64_t* dq_out);
/* The whole attention VJP from one kernel: returns ds as malus_std_attn_bwd,
 * with dq = dq_add + ds @ k, dk = dk_add + ds^T @ q and dv = dv_add + p^T @ dout
 * [bh, t, hs] into *dq_out, *dk_out, *dv_out (all required); an addend handle
 * of 0 adds nothing (the gradient accumulation the tape folds in).  These are
 * the matmul VJPs (tape.rs:460-469) of the two products of the composed
 * attention (nanogpt_modular.ml:57-62). */
int64_t malus_std_attn_bwd_all(int64_t dout, int64_t q, int64_t k, int64_t v, int64_t p, int64_t scale,
                               int32_t causal, int64_t dq_add, int64_t dk_add, int64_t dv_add, int64_t* dq_out,
                               int64_t* dk_out, int64_t* dv_out);
/* Flash attention (online softmax; docs/adr/0029-composed-attention.md:23-33,
 * the fused attention the reference reserves): returns softmax(q @ k^T *
 * scale + causal mask) @ v [bh, t, hs] without forming the [bh, t, t]
 * scores or probabilities (causal 0: no mask); *lse_out (if non-null)
 * receives the row log-sum-exp [bh, t] the backward needs.  t is any
 * multiple of 32, hs 32 or 64; under malus_autocast the products run on
 * the bf16 MFMA.  No reference counterpart as an entry point: the reference
 * composes the same value from matmul and softmax (nanogpt_modular.ml:57-62). */
int64_t malus_std_flash_attn_fwd(int64_t q, int64_t k, int64_t v, int64_t scale, int32_t causal, int64_t* lse_out);
/* Its VJP: dq = dq_add + ..., dk = dk_add + ..., dv = dv_add + ... (the
 * addends may be 0) from dout [bh, t, hs], the forward's inputs, output and
 * lse; P is recomputed.  Returns 0, or -1 with the error set. */
int32_t malus_std_flash_attn_bwd(int64_t dout, int64_t q, int64_t k, int64_t v, int64_t out, int64_t lse,
                                 int64_t scale, int32_t causal, int64_t dq_add, int64_t dk_add, int64_t dv_add,
                                 int64_t* dq_out, int64_t* dk_out, int64_t* dv_out);
int64_t malus_ktimer_collect(const char* cls, double* total_ms, double* total_units);
int malus_device_info(char* name, size_t cap, int* cus, int* clock_khz);
int malus_set_abort_on_error(int on); /* returns the previous setting */
const char* malus_last_error(void);
void malus_clear_error(void);

/* ---- stdlib host functions ------------------------------------------------
 * The .ml host fns of crates/malus-stdlib/stdlib (names prefixed malus_std_),
 * on hand-written gfx950 kernels.  The backward ones are the default BwdSlot
 * entries (codegen-cpu/lib.rs:189-220). */
int64_t malus_std_broadcast_fwd(int32_t op /*0 add,1 sub,2 mul,3 div*/, int64_t a, int64_t b); /* broadcast_binop.ml:82-112 */
int64_t malus_std_broadcast_add_fwd(int64_t a, int64_t b);
int64_t malus_std_broadcast_sub_fwd(int64_t a, int64_t b);
int64_t malus_std_broadcast_mul_fwd(int64_t a, int64_t b);
int64_t malus_std_broadcast_div_fwd(int64_t a, int64_t b);
int64_t malus_std_scalar_op(int32_t op, int64_t a, float s, int32_t scalar_on_right);    /* codegen-gpu/lib.rs:400-418 */
int64_t malus_std_scalar_op_dev(int32_t op, int64_t a, int64_t s1, int32_t scalar_on_right);
int64_t malus_std_unary(int32_t op /*relu,sigmoid,tanh,exp,log,sqrt,abs,gelu*/, int64_t x); /* codegen-gpu/lib.rs:373-390 */
int64_t malus_std_reduce_fwd(int32_t op /*sum,mean,max,var*/, int64_t x, int64_t axis, int64_t keepdim); /* reduce_*.ml */
int64_t malus_std_reduce_all_sum_fwd(int64_t x);                             /* reduce_all.ml:9-12 */
int64_t malus_std_softmax_fwd(int64_t x, int64_t axis);                      /* softmax.ml:30-40 */
int64_t malus_std_layernorm_fwd(int64_t x, int64_t axis, int64_t* var_out);  /* layernorm.ml:59-72 */
int64_t malus_std_gelu_fwd(int64_t x);                                       /* gelu.ml:12-14 */
/* No reference counterpart (docs/adr/0037-bf16-autocast.md:30: f32<->bf16
 * conversion kernels join the stdlib): x converted to dtype (0 = F32,
 * 2 = BF16; round to nearest even into bf16, exact into f32). */
int64_t malus_std_cast(int64_t x, int32_t dtype);
int64_t malus_std_cross_entropy_fwd(int64_t logits, int64_t targets, int64_t* probs_out); /* cross_entropy.ml:18-28 */
int64_t malus_std_embedding_fwd(int64_t weight, int64_t indices);            /* embedding.ml:18-23 */
int64_t malus_std_transpose_2d_fwd(int64_t x);                               /* permute.ml:21-25 */
int64_t malus_std_permute_3d_fwd(int64_t x, int64_t p0, int64_t p1, int64_t p2); /* permute.ml:62-67 */
int64_t malus_std_permute_nd_fwd(int64_t x, int64_t p0, int64_t p1, int64_t p2, int64_t p3, int64_t p4,
                                 int64_t p5, int64_t p6, int64_t p7);        /* permute.ml:107-126 */
int64_t malus_std_scale_fwd(int64_t x, float c);                             /* unary_bwd.ml:10-12 */
int64_t malus_std_fill_like_fwd(int64_t x, float c);                         /* unary_bwd.ml:20-22 */
int64_t malus_std_eq_fwd(int64_t a, int64_t b);                              /* unary_bwd.ml:32-34 */
int64_t malus_std_expand_axis_fwd(int64_t small, int64_t x_template, int64_t axis); /* reduce_bwd.ml:22-38 */
int64_t malus_std_sum_to_shape_bwd(int64_t dout, int64_t target);            /* elementwise_bwd.ml:8-22 */
int64_t malus_std_add_bwd_a(int64_t dout, int64_t a);                        /* elementwise_bwd.ml:25-26 */
int64_t malus_std_add_bwd_b(int64_t dout, int64_t b);                        /* elementwise_bwd.ml:28-29 */
int64_t malus_std_sub_bwd_a(int64_t dout, int64_t a);                        /* elementwise_bwd.ml:32-33 */
int64_t malus_std_sub_bwd_b(int64_t dout, int64_t b);                        /* elementwise_bwd.ml:35-37 */
int64_t malus_std_mul_bwd_a(int64_t dout, int64_t a, int64_t b);             /* elementwise_bwd.ml:41-43 */
int64_t malus_std_mul_bwd_b(int64_t dout, int64_t a, int64_t b);             /* elementwise_bwd.ml:45-47 */
int64_t malus_std_div_bwd_a(int64_t dout, int64_t a, int64_t b);             /* elementwise_bwd.ml:51-53 */
int64_t malus_std_div_bwd_b(int64_t dout, int64_t a, int64_t b);             /* elementwise_bwd.ml:55-60 */
int64_t malus_std_sigmoid_bwd(int64_t s, int64_t dout);                      /* unary_bwd.ml:42-44 */
int64_t malus_std_relu_bwd(int64_t x, int64_t dout);                         /* unary_bwd.ml:54-56 */
int64_t malus_std_tanh_bwd(int64_t t, int64_t dout);                         /* unary_bwd.ml:64-66 */
int64_t malus_std_sqrt_bwd(int64_t s, int64_t dout);                         /* unary_bwd.ml:73-75 */
int64_t malus_std_abs_bwd(int64_t x, int64_t dout);                          /* unary_bwd.ml:89-91 */
int64_t malus_std_sum_bwd(int64_t x, int64_t dout);                          /* reduce_bwd.ml:74-76 */
int64_t malus_std_reduce_sum_axis_bwd(int64_t x, int64_t dout, int64_t axis);   /* reduce_bwd.ml:41-42 */
int64_t malus_std_reduce_mean_axis_bwd(int64_t x, int64_t dout, int64_t axis);  /* reduce_bwd.ml:45-51 */
int64_t malus_std_reduce_max_axis_bwd(int64_t x, int64_t y, int64_t dout, int64_t axis); /* reduce_bwd.ml:54-58 */
int64_t malus_std_reduce_var_axis_bwd(int64_t x, int64_t dout, int64_t axis);   /* reduce_bwd.ml:61-71 */
int64_t malus_std_softmax_bwd(int64_t s, int64_t dout, int64_t axis);           /* transformer_bwd.ml:15-20 */
int64_t malus_std_layernorm_bwd(int64_t y, int64_t var, int64_t dout, int64_t axis); /* tape.rs:1162-1186 */
int64_t malus_std_gelu_bwd(int64_t x, int64_t dout);                         /* transformer_bwd.ml:50-52 */
int64_t malus_std_cross_entropy_bwd(int64_t probs, int64_t targets, int64_t dout); /* transformer_bwd.ml:67-75 */
int64_t malus_std_embedding_bwd(int64_t weight, int64_t indices, int64_t dout);    /* transformer_bwd.ml:93-98 */
int64_t malus_std_matmul_bwd_a(int64_t a, int64_t b, int64_t dout);          /* matmul_bwd.ml:15-19 */
int64_t malus_std_matmul_bwd_b(int64_t a, int64_t b, int64_t dout);          /* matmul_bwd.ml:21-29 */
/* examples/nanogpt_modular.ml:97-108 fused into one pass; returns the new
 * parameter, *m_out / *v_out the new moments. */
int64_t malus_std_adam_l2(int64_t p, int64_t g, int64_t m, int64_t v, float lr, float b1, float b2, float eps,
                          float wd, int64_t t, int64_t* m_out, int64_t* v_out);

/* ---- workload drivers (the examples' programs replayed through this ABI) - */
void* malus_gpt_create(int vocab, int block, int n_embd, int n_head, int n_layer, int batch, float lr, float beta1,
                       float beta2, float eps, float wd); /* nanogpt_modular.ml:138-164 */
void malus_gpt_free(void* g);
int malus_gpt_nparams(void* g);
int64_t malus_gpt_param(void* g, int i);              /* borrowed */
int64_t malus_gpt_moment(void* g, int i, int which);  /* borrowed; which 0 = m, 1 = v */
void malus_gpt_set_fused_optimizer(void* g, int on);
/* Attention of the model: 0 automatic (flash attention under
 * malus_autocast, and with split f32 GEMM products at T >= 256; else the
 * row-register fused kernel where its shapes are built, else flash, else
 * composed), 1 flash attention, 2 the row-register kernel, 3 the composed
 * ops.  Returns 0 or -1. */
int malus_gpt_set_attention(void* gpt, int mode);
/* 1 (default): forward fusions (attention scale+mask+softmax, residual adds in GEMM epilogues); 0: separate ops (same values and tape). */
void malus_gpt_set_fused_forward(void* g, int on);
/* No reference counterpart (the autocast storage policy of
 * docs/adr/0037-bf16-autocast.md:8).  1 (default): under malus_autocast the
 * activations read only as bf16 MFMA operands (the layernorm-scale outputs,
 * gelu(h), the GELU VJP's dh and, with flash attention, q, k, v and their
 * gradients) are stored in bf16, and the GEMMs read bf16 copies of the block
 * weights refreshed at each forward; the step's values are the same as with
 * 0 (f32 storage), in half the bytes.  With split f32 products
 * (malus_gemm_set_f32_split) the block weights get split copies instead
 * (the three bf16 planes of their pieces, refreshed at each forward), which
 * the forward GEMMs read as B without splitting it; the same values as
 * with 0. */
void malus_gpt_set_bf16_activations(void* g, int on);
int64_t malus_gpt_forward_loss(void* g, int64_t toks, int64_t targets); /* nanogpt_modular.ml:75-91 + cross_entropy */
int64_t malus_gpt_logits(void* g, int64_t toks);
void malus_gpt_zero_grad(void* g);
void malus_gpt_optimizer_step(void* g, int64_t t);    /* nanogpt_modular.ml:186-188 */
int64_t malus_gpt_step(void* g, int64_t toks, int64_t targets, int64_t t); /* nanogpt_modular.ml:167-189 */
/* No reference counterpart: the whole training step as a HIP graph (the
 * "optionally hipGraph-captured train steps" of the north star).  create runs
 * step t eagerly (its loss in *loss_out) and captures the step; each
 * graph_step replays it for step t on new token/target ids (copied from
 * pinned host memory by the graph's own nodes) and returns the loss tensor
 * (the same device buffer every step).  Parameters are updated in place; the
 * values equal malus_gpt_step's.  Free the graph before the model. */
void* malus_gpt_graph_create(void* gpt, const int32_t* x, const int32_t* y, int64_t t, int64_t* loss_out);
int64_t malus_gpt_graph_step(void* graph, const int32_t* x, const int32_t* y, int64_t t);
/* The same graph with each step's ids drawn on the device by a kernel node
 * of the step itself: x[i] = rand_int(V) with call index x_call + i, y[i]
 * with y_call + i (the ids malus_rand_tokens_device draws), so batch
 * construction is part of the replayed step. */
void* malus_gpt_graph_create_drawn(void* gpt, uint64_t x_call, uint64_t y_call, int64_t t, int64_t* loss_out);
int64_t malus_gpt_graph_step_drawn(void* graph, uint64_t x_call, uint64_t y_call, int64_t t);
void malus_gpt_graph_free(void* graph);
size_t malus_gpt_graph_nodes(void* graph);
/* No reference counterpart (a checkpoint format is deferred in the
 * reference, CLAUDE.md:70): the model's parameters and AdamW moments as a
 * SafeTensors file, with the step in its metadata.  save returns 0; load
 * checks names, dtypes and shapes against the model and returns the step
 * (both -1 in return-error mode). */
int malus_gpt_save(void* gpt, const char* path, int64_t step);
int64_t malus_gpt_load(void* gpt, const char* path);
float malus_xor_run(int steps, float lr, uint64_t sigmoid_backward_id, float* loss_at, float* preds,
                    float* params); /* examples/xor.ml */

#ifdef __cplusplus
}
#endif
#endif /* MALUS_HIP_H */
