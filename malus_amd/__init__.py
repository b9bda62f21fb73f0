"""malus_amd — MI355X (gfx950) backend for the malus runtime ABI.

The product is ``libmalus_hip.so``: a C-ABI shared library exporting the
malus runtime symbols (include/malus_hip.h).  This module loads it with
ctypes for tests and benchmarks.  There is no CPU fallback: if the library
is missing or no HIP device is present, calls fail loudly.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libmalus_hip.so"

F32, BF16, I32, I64 = 0, 2, 5, 6
_NP_DTYPE = {F32: np.float32, I32: np.int32, I64: np.int64}
_TAG_OF = {np.dtype(np.float32): F32, np.dtype(np.int32): I32, np.dtype(np.int64): I64}

# op codes shared with the library
ADD, SUB, MUL, DIV = 0, 1, 2, 3
RELU, SIGMOID, TANH, EXP, LOG, SQRT, ABS, GELU = range(8)
R_SUM, R_MEAN, R_MAX, R_VAR = range(4)

_i64, _i32, _u64, _f32, _sz, _vp = C.c_int64, C.c_int32, C.c_uint64, C.c_float, C.c_size_t, C.c_void_p
_P = C.POINTER

# name: (restype, argtypes)
SIGNATURES = {
    # tensors (metal.rs)
    "malus_init": (None, []),
    "tensor_alloc_gpu": (_i64, [_i32, _P(_sz), _sz, _vp]),
    "tensor_alloc_zeros_gpu": (_i64, [_P(_sz), _sz]),
    "tensor_alloc_ones_gpu": (_i64, [_P(_sz), _sz]),
    "tensor_retain": (None, [_i64]),
    "tensor_release": (None, [_i64]),
    "tensor_free": (None, [_i64]),
    "tensor_print": (None, [_i64]),
    "tensor_len": (_i64, [_i64]),
    "tensor_ndim": (_i64, [_i64]),
    "tensor_dim": (_i64, [_i64, _i64]),
    "malus_tensor_dtype": (_i32, [_i64]),
    "malus_tensor_shape": (None, [_i64, _P(_sz)]),
    "malus_tensor_get_f32": (_f32, [_i64, _i64]),
    "malus_tensor_read": (None, [_i64, _vp, _sz]),
    "malus_tensor_write": (None, [_i64, _vp, _sz]),
    "malus_tensor_device_ptr": (_vp, [_i64]),
    "malus_format_f32": (_sz, [_f32, C.c_char_p, _sz]),
    "gpu_barrier": (None, []),
    "malus_flush_if_pending": (None, [_i64]),
    "tensor_is_pending": (C.c_int, [_i64]),
    "tensor_matmul": (_i64, [_i64, _i64]),
    "tensor_reshape": (_i64, [_i64, _P(_sz), _sz]),
    "tensor_permute": (_i64, [_i64, _P(_sz), _sz]),
    "tensor_causal_mask": (_i64, [_i64]),
    "tensor_randn": (_i64, [_P(_sz), _sz]),
    "malus_rand_uniform": (_f32, []),
    "malus_rand_int": (_i64, [_i64]),
    "malus_rng_get_counter": (_u64, []),
    "malus_rng_set_counter": (None, [_u64]),
    "kernel_dispatch": (_i64, [_u64, _P(_i64), _sz]),
    "kernel_dispatch_v2": (_i64, [_u64, _P(_i64), _sz, _P(_sz), _P(_sz), _P(_sz), _sz, _i32, _vp, _sz]),
    "malus_runtime_init": (None, [_P(_u64), _P(C.c_char_p), _sz]),
    "malus_kernel_is_builtin": (C.c_int, [_u64]),
    "malus_rtc_compile": (C.c_size_t, [C.c_char_p, C.c_char_p, C.c_void_p, C.c_size_t, C.c_char_p, C.c_size_t]),
    # buffers (buffer.rs)
    "malus_buffer_i32": (_i64, [_i64]),
    "malus_buffer_get_i32": (_i64, [_i64, _i64]),
    "malus_buffer_set_i32": (None, [_i64, _i64, _i64]),
    "malus_buffer_free": (None, [_i64]),
    "malus_buffer_freeze_i32": (_i64, [_i64]),
    # tape (tape.rs)
    "tape_record_binop": (None, [_i32, _i64, _i64, _i64]),
    "tape_record_unary": (None, [_i32, _i64, _i64]),
    "tape_record_reduce": (None, [_i32, _i64, _i64, _i64, _i64]),
    "tape_record_perm": (None, [_i32, _i64, _i64, _P(_sz), _sz]),
    "tape_record_layernorm": (None, [_i32, _i64, _i64, _i64, _i64]),
    "tape_record_cross_entropy": (None, [_i32, _i64, _i64, _i64, _i64]),
    "tape_record_embedding": (None, [_i32, _i64, _i64, _i64]),
    "tape_register_leaf": (None, [_i64]),
    "tape_pause": (None, []),
    "tape_resume": (None, []),
    "tape_clear": (None, []),
    "tape_get_grad": (_i64, [_i64]),
    "backward": (None, [_i64]),
    "tape_zero_grad": (None, [_P(_i64), _sz]),
    "tape_reset": (None, []),
    "tape_register_backward_fn": (None, [_i32, _sz]),
    "malus_tape_backward_fn": (_sz, [_i32]),
    "malus_tape_len": (_sz, []),
    "malus_tape_registry_lens": (None, [_P(_sz)]),
    # bench / counters / pool
    "bench_enable": (None, []),
    "bench_reset": (None, []),
    "bench_step_begin": (None, []),
    "bench_step_end": (None, []),
    "bench_report": (C.c_int, [_P(C.c_double), _P(C.c_double), _P(C.c_double), _P(_i64)]),
    "malus_bench_record": (None, [C.c_double]),
    "malus_cpu_compute_count": (_i64, []),
    "malus_cpu_compute_reset": (None, []),
    "malus_rc_counts": (None, [_P(_i64)]),
    "malus_rc_reset": (None, []),
    "malus_record_diff": (None, [_f32]),
    "malus_gradcheck_max_diff": (_f32, []),
    "malus_gradcheck_reset": (None, []),
    "malus_pool_stats": (None, [_P(_i64)]),
    "malus_pool_live_bytes": (_i64, []),
    "malus_pool_buckets": (_sz, [_P(_sz), _P(_sz), _sz]),
    "malus_pool_reset": (None, []),
    "malus_set_mem_budget": (None, [_i64]),
    "malus_fail_alloc_after": (None, [_i64]),
    "malus_alloc_histogram": (_sz, [_P(_sz), _P(_u64), _sz]),
    "malus_ktimer_enable": (None, [C.c_int]),
    "malus_gemm_set_tile": (C.c_int, [C.c_int, C.c_int]),
    "malus_gemm_set_split": (None, [C.c_int]),
    "malus_gemm_set_dma": (None, [C.c_int]),
    "malus_gemm_set_f32_split": (C.c_int, [C.c_int]),
    "malus_autocast": (C.c_int, [C.c_int]),
    "malus_std_attn_scores_softmax": (_i64, [_i64, _i64, _i64, _i64, _i32]),
    "malus_std_attn_scores_bwd": (_i64, [_i64, _i64, _i64, _i64, _i32]),
    "malus_std_attn_fwd": (_i64, [_i64, _i64, _i64, _i64, _i64, _i32, _P(_i64)]),
    "malus_std_attn_bwd": (_i64, [_i64, _i64, _i64, _i64, _i64, _i32, _P(_i64)]),
    "malus_std_attn_bwd_all": (_i64, [_i64, _i64, _i64, _i64, _i64, _i64, _i32, _i64, _i64, _i64, _P(_i64), _P(_i64),
                                      _P(_i64)]),
    "malus_std_flash_attn_fwd": (_i64, [_i64, _i64, _i64, _i64, _i32, _P(_i64)]),
    "malus_std_flash_attn_bwd": (_i32, [_i64, _i64, _i64, _i64, _i64, _i64, _i64, _i32, _i64, _i64, _i64,
                                             _P(_i64), _P(_i64), _P(_i64)]),
    "malus_ktimer_collect": (_i64, [C.c_char_p, _P(C.c_double), _P(C.c_double)]),
    "malus_device_info": (C.c_int, [C.c_char_p, _sz, _P(C.c_int), _P(C.c_int)]),
    "malus_set_abort_on_error": (C.c_int, [C.c_int]),
    "malus_last_error": (C.c_char_p, []),
    "malus_clear_error": (None, []),
    # stdlib host fns
    "malus_std_broadcast_fwd": (_i64, [_i32, _i64, _i64]),
    "malus_std_scalar_op": (_i64, [_i32, _i64, _f32, _i32]),
    "malus_std_scalar_op_dev": (_i64, [_i32, _i64, _i64, _i32]),
    "malus_std_unary": (_i64, [_i32, _i64]),
    "malus_std_reduce_fwd": (_i64, [_i32, _i64, _i64, _i64]),
    "malus_std_reduce_all_sum_fwd": (_i64, [_i64]),
    "malus_std_softmax_fwd": (_i64, [_i64, _i64]),
    "malus_std_layernorm_fwd": (_i64, [_i64, _i64, _P(_i64)]),
    "malus_std_gelu_fwd": (_i64, [_i64]),
    "malus_std_cross_entropy_fwd": (_i64, [_i64, _i64, _P(_i64)]),
    "malus_std_embedding_fwd": (_i64, [_i64, _i64]),
    "malus_std_transpose_2d_fwd": (_i64, [_i64]),
    "malus_std_permute_3d_fwd": (_i64, [_i64, _i64, _i64, _i64]),
    "malus_std_permute_nd_fwd": (_i64, [_i64] + [_i64] * 8),
    "malus_std_scale_fwd": (_i64, [_i64, _f32]),
    "malus_std_fill_like_fwd": (_i64, [_i64, _f32]),
    "malus_std_eq_fwd": (_i64, [_i64, _i64]),
    "malus_std_expand_axis_fwd": (_i64, [_i64, _i64, _i64]),
    "malus_std_reduce_sum_axis_bwd": (_i64, [_i64, _i64, _i64]),
    "malus_std_reduce_mean_axis_bwd": (_i64, [_i64, _i64, _i64]),
    "malus_std_reduce_max_axis_bwd": (_i64, [_i64, _i64, _i64, _i64]),
    "malus_std_reduce_var_axis_bwd": (_i64, [_i64, _i64, _i64]),
    "malus_std_sum_to_shape_bwd": (_i64, [_i64, _i64]),
    "malus_std_mul_bwd_a": (_i64, [_i64, _i64, _i64]),
    "malus_std_mul_bwd_b": (_i64, [_i64, _i64, _i64]),
    "malus_std_softmax_bwd": (_i64, [_i64, _i64, _i64]),
    "malus_std_layernorm_bwd": (_i64, [_i64, _i64, _i64, _i64]),
    "malus_std_gelu_bwd": (_i64, [_i64, _i64]),
    "malus_std_cross_entropy_bwd": (_i64, [_i64, _i64, _i64]),
    "malus_std_embedding_bwd": (_i64, [_i64, _i64, _i64]),
    "malus_std_matmul_bwd_a": (_i64, [_i64, _i64, _i64]),
    "malus_std_matmul_bwd_b": (_i64, [_i64, _i64, _i64]),
    "malus_std_sigmoid_bwd": (_i64, [_i64, _i64]),
    "malus_std_relu_bwd": (_i64, [_i64, _i64]),
    "malus_std_tanh_bwd": (_i64, [_i64, _i64]),
    "malus_std_sqrt_bwd": (_i64, [_i64, _i64]),
    "malus_std_abs_bwd": (_i64, [_i64, _i64]),
    "malus_std_sum_bwd": (_i64, [_i64, _i64]),
    "malus_std_adam_l2": (_i64, [_i64, _i64, _i64, _i64, _f32, _f32, _f32, _f32, _f32, _i64, _P(_i64), _P(_i64)]),
    # workload drivers
    "malus_gpt_create": (_vp, [C.c_int] * 6 + [_f32] * 5),
    "malus_gpt_free": (None, [_vp]),
    "malus_gpt_nparams": (C.c_int, [_vp]),
    "malus_gpt_param": (_i64, [_vp, C.c_int]),
    "malus_gpt_moment": (_i64, [_vp, C.c_int, C.c_int]),
    "malus_gpt_set_fused_optimizer": (None, [_vp, C.c_int]),
    "malus_gpt_set_attention": (C.c_int, [_vp, C.c_int]),
    "malus_gpt_set_fused_forward": (None, [_vp, C.c_int]),
    "malus_std_cast": (_i64, [_i64, C.c_int32]),
    "malus_gpt_set_bf16_activations": (None, [_vp, C.c_int]),
    "malus_tape_set_fused_vjps": (None, [C.c_int]),
    "malus_gpt_forward_loss": (_i64, [_vp, _i64, _i64]),
    "malus_gpt_logits": (_i64, [_vp, _i64]),
    "malus_gpt_zero_grad": (None, [_vp]),
    "malus_gpt_optimizer_step": (None, [_vp, _i64]),
    "malus_gpt_step": (_i64, [_vp, _i64, _i64, _i64]),
    "malus_xor_run": (_f32, [C.c_int, _f32, _u64, _P(_f32), _P(_f32), _P(_f32)]),
    "malus_gpt_graph_create": (_vp, [_vp, _P(_i32), _P(_i32), _i64, _P(_i64)]),
    "malus_gpt_graph_step": (_i64, [_vp, _P(_i32), _P(_i32), _i64]),
    "malus_gpt_graph_create_drawn": (_vp, [_vp, _u64, _u64, _i64, _P(_i64)]),
    "malus_gpt_graph_step_drawn": (_i64, [_vp, _u64, _u64, _i64]),
    "malus_gpt_graph_free": (None, [_vp]),
    "malus_gpt_graph_nodes": (_sz, [_vp]),
    "malus_gpt_save": (C.c_int, [_vp, C.c_char_p, _i64]),
    "malus_gpt_load": (_i64, [_vp, C.c_char_p]),
    "malus_randn_device": (_i64, [_P(_sz), _sz]),
    "malus_batch_windows": (None, [_i64, _i64, _i64, _P(_i64), _P(_i64), _P(C.c_int32)]),
    "malus_rand_tokens_device": (_i64, [C.c_uint64, _sz, _i64]),
    "malus_std_reduce_noalloc": (C.c_int, [_i32, _vp, _P(_sz), _sz, _i64, _vp]),
    "malus_compile_kernels": (_vp, [C.c_char_p, _P(C.c_char_p), _sz, C.c_int]),
    "malus_registry_len": (_sz, [_vp]),
    "malus_registry_id": (_u64, [_vp, _sz]),
    "malus_registry_name": (C.c_char_p, [_vp, _sz]),
    "malus_registry_source": (C.c_char_p, [_vp, _sz]),
    "malus_registry_lookup": (C.c_int, [_vp, C.c_char_p, _P(_u64)]),
    "malus_registry_free": (None, [_vp]),
}

_lib = None


def lib():
    """Load libmalus_hip.so (built in-tree by ``python -m malus_amd.build``)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built; run `python -m malus_amd.build` (no CPU fallback exists)")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def sizes(vals) -> "C.Array":
    vals = list(vals)
    return (_sz * max(1, len(vals)))(*vals)


def handles(vals) -> "C.Array":
    vals = list(vals)
    return (_i64 * max(1, len(vals)))(*vals)


class Runtime:
    """Convenience wrapper over the C ABI for tests and benchmarks."""

    def __init__(self):
        self.L = lib()
        self.L.malus_init()

    # -- tensors --------------------------------------------------------------
    def tensor(self, arr) -> int:
        a = np.ascontiguousarray(arr)
        if a.dtype not in _TAG_OF:
            a = a.astype(np.float32)
        tag = _TAG_OF[a.dtype]
        shape = a.shape if a.ndim else (1,)
        return self.L.tensor_alloc_gpu(tag, sizes(shape), len(shape), a.ctypes.data_as(_vp))

    def shape(self, h: int) -> tuple:
        nd = self.L.tensor_ndim(h)
        buf = (_sz * 8)()
        self.L.malus_tensor_shape(h, buf)
        return tuple(buf[i] for i in range(nd))

    def numpy(self, h: int) -> np.ndarray:
        """The tensor's values on the host; a bf16 tensor comes back as the
        float32 array of its (exactly representable) values."""
        tag = self.L.malus_tensor_dtype(h)
        shp = self.shape(h)
        if tag == BF16:
            raw = np.empty(shp, dtype=np.uint16)
            if raw.size:
                self.L.malus_tensor_read(h, raw.ctypes.data_as(_vp), raw.nbytes)
            return (raw.astype(np.uint32) << 16).view(np.float32)
        out = np.empty(shp, dtype=_NP_DTYPE[tag])
        if out.size:
            self.L.malus_tensor_read(h, out.ctypes.data_as(_vp), out.nbytes)
        return out

    def bf16(self, arr) -> int:
        """A bf16 tensor of arr's values rounded to nearest even (the
        stdlib's malus_std_cast of an f32 upload)."""
        h = self.tensor(np.asarray(arr, dtype=np.float32))
        out = self.L.malus_std_cast(h, BF16)
        self.free(h)
        return out

    def free(self, *hs):
        for h in hs:
            if h:
                self.L.tensor_free(h)

    def last_error(self) -> str:
        e = self.L.malus_last_error()
        return e.decode() if e else ""


class KernelRegistry:
    """compile_kernels' output (the emitter's id -> HIP source map, plus name
    -> id), read out of the library's registry."""

    def __init__(self, entries):
        self.entries = entries  # [(name, id, source)] in id order
        self.ids = {n: i for n, i, _ in entries}
        self.sources = {n: s for n, _, s in entries}

    def init_args(self):
        """(ids, sources, n) for malus_runtime_init."""
        n = len(self.entries)
        ids = (_u64 * max(1, n))(*[i for _, i, _ in self.entries])
        srcs = (C.c_char_p * max(1, n))(*[s.encode() for _, _, s in self.entries])
        return ids, srcs, n


def compile_kernels(program: str, builtins=(), tags: bool = False) -> KernelRegistry:
    """Lower the `kernel` items of malus source `program` (and the named
    synthesized builtins) to HIP with the library's emitter.  Raises
    RuntimeError with the emitter's message on a bad program.  Needs no GPU."""
    L = lib()
    names = [b.encode() for b in builtins]
    arr = (C.c_char_p * max(1, len(names)))(*names)
    prev = L.malus_set_abort_on_error(0)
    try:
        r = L.malus_compile_kernels(program.encode(), arr, len(names), 1 if tags else 0)
        if not r:
            msg = L.malus_last_error()
            L.malus_clear_error()
            raise RuntimeError(msg.decode() if msg else "malus_compile_kernels failed")
    finally:
        L.malus_set_abort_on_error(prev)
    try:
        entries = [(L.malus_registry_name(r, i).decode(), int(L.malus_registry_id(r, i)),
                    L.malus_registry_source(r, i).decode()) for i in range(L.malus_registry_len(r))]
    finally:
        L.malus_registry_free(r)
    return KernelRegistry(entries)


class autocast:
    """`with autocast():` -- the scope of docs/adr/0037-bf16-autocast.md:5-12
    over malus_autocast: GEMMs in bf16 with f32 accumulation inside the
    block, the previous state restored on exit (nested blocks compose)."""

    def __init__(self, enabled: bool = True):
        self.enabled = enabled
        self._prev = 0

    def __enter__(self):
        self._prev = lib().malus_autocast(1 if self.enabled else 0)
        return self

    def __exit__(self, *exc):
        lib().malus_autocast(self._prev)
        return False

