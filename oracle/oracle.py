"""ctypes binding of the CPU oracle (oracle/malus_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker.  Nothing in malus_amd imports it.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libmalus_oracle.so"

ADD, SUB, MUL, DIV = 0, 1, 2, 3
RELU, SIGMOID, TANH, EXP, LOG, SQRT, ABS, GELU = range(8)
R_SUM, R_MEAN, R_MAX, R_VAR = range(4)

_f = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int32)
_szp = C.POINTER(C.c_size_t)
_u32p = C.POINTER(C.c_uint32)


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


_L = None


def lib():
    global _L
    if _L is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        sig = {
            "or_philox4x32_10": (None, [_u32p, _u32p, _u32p]),
            "or_randn": (None, [C.c_uint64, C.c_size_t, _f]),
            "or_rand_uniform": (C.c_float, [C.c_uint64]),
            "or_rand_int": (C.c_int64, [C.c_uint64, C.c_int64]),
            "or_rand_tokens": (None, [C.c_uint64, C.c_size_t, C.c_int64, _i32p]),
            "or_broadcast_fwd": (None, [C.c_int, _f, _szp, C.c_int, _f, _szp, C.c_int, _f, _szp, C.POINTER(C.c_int)]),
            "or_scalar_op": (None, [C.c_int, C.c_int, _f, C.c_size_t, C.c_float, _f]),
            "or_unary": (None, [C.c_int, _f, C.c_size_t, _f]),
            "or_reduce_axis": (None, [C.c_int, _f, _szp, C.c_int, C.c_int, _f]),
            "or_sum_all": (C.c_float, [_f, C.c_size_t]),
            "or_reduce_axis_bwd": (None, [C.c_int, _f, _f, _f, _szp, C.c_int, C.c_int, _f]),
            "or_softmax_axis": (None, [_f, _szp, C.c_int, C.c_int, _f]),
            "or_layernorm_axis": (None, [_f, _szp, C.c_int, C.c_int, _f, _f]),
            "or_cross_entropy": (C.c_float, [_f, C.c_size_t, C.c_size_t, _i32p, _f]),
            "or_embedding": (None, [_f, C.c_size_t, C.c_size_t, _i32p, C.c_size_t, _f]),
            "or_causal_mask": (None, [C.c_size_t, _f]),
            "or_permute": (None, [_f, _szp, C.c_int, _szp, _f]),
            "or_matmul": (None, [_f, _szp, C.c_int, _f, _szp, C.c_int, _f]),
            "or_sum_to_shape": (None, [_f, _szp, C.c_int, _szp, C.c_int, _f]),
            "or_unary_bwd": (None, [C.c_int, _f, _f, C.c_size_t, _f]),
            "or_softmax_bwd": (None, [_f, _f, _szp, C.c_int, C.c_int, _f]),
            "or_layernorm_bwd": (None, [_f, _f, _f, _szp, C.c_int, C.c_int, _f]),
            "or_cross_entropy_bwd": (None, [_f, C.c_size_t, C.c_size_t, _i32p, C.c_float, _f]),
            "or_embedding_bwd": (None, [_f, _i32p, C.c_size_t, C.c_size_t, C.c_size_t, _f]),
            "or_adam_l2_update": (None, [_f, _f, _f, _f, C.c_size_t] + [C.c_float] * 5 + [C.c_int64]),
            "or_xor_train": (C.c_float, [C.c_int, C.c_float, _f, _f, _f]),
            "or_gpt_create": (C.c_void_p, [C.c_int] * 6 + [C.c_uint64] + [C.c_float] * 5),
            "or_gpt_free": (None, [C.c_void_p]),
            "or_gpt_nparams": (C.c_int, [C.c_void_p]),
            "or_gpt_param_len": (C.c_size_t, [C.c_void_p, C.c_int]),
            "or_gpt_get_param": (None, [C.c_void_p, C.c_int, _f]),
            "or_gpt_get_grad": (None, [C.c_void_p, C.c_int, _f]),
            "or_gpt_set_param": (None, [C.c_void_p, C.c_int, _f]),
            "or_gpt_get_moment": (None, [C.c_void_p, C.c_int, C.c_int, _f]),
            "or_gpt_set_moment": (None, [C.c_void_p, C.c_int, C.c_int, _f]),
            "or_gpt_loss_and_grads": (C.c_float, [C.c_void_p, _i32p, _i32p, _f]),
            "or_gpt_step": (C.c_float, [C.c_void_p, _i32p, _i32p, C.c_int64]),
            "or_set_threads": (None, [C.c_int]),
            "or_get_threads": (C.c_int, []),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _L = L
    return _L


def _fp(a: np.ndarray):
    return a.ctypes.data_as(_f)


def _sz(vals):
    vals = list(vals)
    return (C.c_size_t * max(1, len(vals)))(*vals)


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def philox(ctr, key):
    c = (C.c_uint32 * 4)(*ctr)
    k = (C.c_uint32 * 2)(*key)
    o = (C.c_uint32 * 4)()
    lib().or_philox4x32_10(c, k, o)
    return list(o)


def randn(call_idx: int, shape) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, np.float32)
    lib().or_randn(call_idx, n, _fp(out))
    return out.reshape(shape)


def rand_tokens(call_idx: int, n: int, vocab: int) -> np.ndarray:
    out = np.empty(n, np.int32)
    lib().or_rand_tokens(call_idx, n, vocab, out.ctypes.data_as(_i32p))
    return out


def broadcast(op, a, b):
    a, b = f32(a), f32(b)
    ash = a.shape or (1,)
    bsh = b.shape or (1,)
    nd = max(len(ash), len(bsh))
    out = np.empty(int(np.prod(np.broadcast_shapes(ash, bsh))), np.float32)
    osh = (C.c_size_t * 8)()
    ond = C.c_int()
    lib().or_broadcast_fwd(op, _fp(a), _sz(ash), len(ash), _fp(b), _sz(bsh), len(bsh), _fp(out), osh, C.byref(ond))
    return out.reshape(tuple(osh[i] for i in range(ond.value)))


def scalar_op(op, a, s, scalar_on_right=True):
    a = f32(a)
    out = np.empty_like(a)
    lib().or_scalar_op(op, int(scalar_on_right), _fp(a), a.size, float(s), _fp(out))
    return out


def unary(op, a):
    a = f32(a)
    out = np.empty_like(a)
    lib().or_unary(op, _fp(a), a.size, _fp(out))
    return out


def unary_bwd(op, xy, dout):
    xy, dout = f32(xy), f32(dout)
    out = np.empty_like(xy)
    lib().or_unary_bwd(op, _fp(xy), _fp(dout), xy.size, _fp(out))
    return out


def reduce_axis(op, x, axis, keepdim=False):
    x = f32(x)
    ax = axis % x.ndim
    out_shape = list(x.shape)
    if keepdim:
        out_shape[ax] = 1
    else:
        out_shape.pop(ax)
    out = np.empty(int(np.prod(out_shape)) if out_shape else 1, np.float32)
    lib().or_reduce_axis(op, _fp(x), _sz(x.shape), x.ndim, axis, _fp(out))
    return out.reshape(out_shape) if out_shape else out


def reduce_axis_bwd(op, x, dout, axis, y=None):
    """VJP of reduce_axis (tape.rs:1085-1145); y = the forward output (max only)."""
    x = f32(x)
    ax = axis % x.ndim
    dout = f32(dout).ravel()
    y = f32(y).ravel() if y is not None else np.zeros(dout.size, np.float32)
    out = np.empty(x.shape, np.float32)
    lib().or_reduce_axis_bwd(op, _fp(x), _fp(y), _fp(dout), _sz(x.shape), x.ndim, ax, _fp(out))
    return out


def sum_all(x):
    x = f32(x)
    return lib().or_sum_all(_fp(x), x.size)


def softmax(x, axis):
    x = f32(x)
    out = np.empty_like(x)
    lib().or_softmax_axis(_fp(x), _sz(x.shape), x.ndim, axis, _fp(out))
    return out


def layernorm(x, axis):
    x = f32(x)
    out = np.empty_like(x)
    vs = list(x.shape)
    vs[axis % x.ndim] = 1
    var = np.empty(vs, np.float32)
    lib().or_layernorm_axis(_fp(x), _sz(x.shape), x.ndim, axis, _fp(out), _fp(var))
    return out, var


def cross_entropy(logits, targets):
    logits = f32(logits)
    t = np.ascontiguousarray(targets, dtype=np.int32)
    probs = np.empty_like(logits)
    loss = lib().or_cross_entropy(_fp(logits), logits.shape[0], logits.shape[1], t.ctypes.data_as(_i32p), _fp(probs))
    return np.float32(loss), probs


def embedding(w, idx):
    w = f32(w)
    i = np.ascontiguousarray(idx, dtype=np.int32)
    out = np.empty((i.size, w.shape[1]), np.float32)
    lib().or_embedding(_fp(w), w.shape[0], w.shape[1], i.ctypes.data_as(_i32p), i.size, _fp(out))
    return out


def causal_mask(t):
    out = np.empty((t, t), np.float32)
    lib().or_causal_mask(t, _fp(out))
    return out


def permute(x, perm):
    x = f32(x)
    out = np.empty(tuple(x.shape[p] for p in perm), np.float32)
    lib().or_permute(_fp(x), _sz(x.shape), x.ndim, _sz(perm), _fp(out))
    return out


def matmul(a, b):
    a, b = f32(a), f32(b)
    if a.ndim == 3 and b.ndim == 3:
        shape = (a.shape[0], a.shape[1], b.shape[2])
    elif a.ndim == 3:
        shape = (a.shape[0], a.shape[1], b.shape[1])
    else:
        shape = (a.shape[0], b.shape[1])
    out = np.empty(shape, np.float32)
    lib().or_matmul(_fp(a), _sz(a.shape), a.ndim, _fp(b), _sz(b.shape), b.ndim, _fp(out))
    return out


def bf16_round(a):
    """f32 -> nearest bf16 (ties to even), returned as f32: the operand
    rounding of the autocast matmul policy (docs/adr/0037-bf16-autocast.md:5-12,
    "matmuls ... compute in bfloat").  bf16 keeps the top 16 bits of the f32
    pattern; finite inputs only."""
    u = f32(a).view(np.uint32).astype(np.uint64)
    r = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return r.astype(np.uint32).view(np.float32)


def sum_to_shape(g, target_shape):
    g = f32(g)
    out = np.empty(target_shape, np.float32)
    lib().or_sum_to_shape(_fp(g), _sz(g.shape), g.ndim, _sz(target_shape), len(target_shape), _fp(out))
    return out


def softmax_bwd(s, dout, axis):
    s, dout = f32(s), f32(dout)
    out = np.empty_like(s)
    lib().or_softmax_bwd(_fp(s), _fp(dout), _sz(s.shape), s.ndim, axis, _fp(out))
    return out


def layernorm_bwd(y, var, dout, axis):
    y, var, dout = f32(y), f32(var), f32(dout)
    out = np.empty_like(y)
    lib().or_layernorm_bwd(_fp(y), _fp(var), _fp(dout), _sz(y.shape), y.ndim, axis, _fp(out))
    return out


def cross_entropy_bwd(probs, targets, dout0):
    probs = f32(probs)
    t = np.ascontiguousarray(targets, dtype=np.int32)
    out = np.empty_like(probs)
    lib().or_cross_entropy_bwd(_fp(probs), probs.shape[0], probs.shape[1], t.ctypes.data_as(_i32p), float(dout0), _fp(out))
    return out


def embedding_bwd(dout, idx, vocab):
    dout = f32(dout)
    i = np.ascontiguousarray(idx, dtype=np.int32)
    out = np.empty((vocab, dout.shape[1]), np.float32)
    lib().or_embedding_bwd(_fp(dout), i.ctypes.data_as(_i32p), i.size, dout.shape[1], vocab, _fp(out))
    return out


def adam_l2(p, g, m, v, lr, b1, b2, eps, wd, t):
    p, g, m, v = (f32(x).copy() for x in (p, g, m, v))
    lib().or_adam_l2_update(_fp(p), _fp(g), _fp(m), _fp(v), p.size, lr, b1, b2, eps, wd, t)
    return p, m, v


def xor_train(steps=10000, lr=1.5):
    loss_at = np.zeros(6, np.float32)
    preds = np.zeros(4, np.float32)
    params = np.zeros(33, np.float32)
    loss = lib().or_xor_train(steps, lr, _fp(loss_at), _fp(preds), _fp(params))
    return np.float32(loss), loss_at, preds, params


class Gpt:
    """Oracle nanoGPT (examples/nanogpt_modular.ml, L blocks / H heads)."""

    def __init__(self, V, T, C, H, L, B, rng_call_idx=0, lr=1e-3, b1=0.9, b2=0.99, eps=1e-8, wd=0.1):
        self.cfg = dict(V=V, T=T, C=C, H=H, L=L, B=B)
        self.h = lib().or_gpt_create(V, T, C, H, L, B, rng_call_idx, lr, b1, b2, eps, wd)

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_gpt_free(self.h)
            self.h = None

    @property
    def nparams(self):
        return lib().or_gpt_nparams(self.h)

    def param(self, i):
        out = np.empty(lib().or_gpt_param_len(self.h, i), np.float32)
        lib().or_gpt_get_param(self.h, i, _fp(out))
        return out

    def grad(self, i):
        out = np.empty(lib().or_gpt_param_len(self.h, i), np.float32)
        lib().or_gpt_get_grad(self.h, i, _fp(out))
        return out

    def set_param(self, i, values):
        v = f32(values).ravel()
        assert v.size == lib().or_gpt_param_len(self.h, i)
        lib().or_gpt_set_param(self.h, i, _fp(v))

    def moment(self, i, which):
        out = np.empty(lib().or_gpt_param_len(self.h, i), np.float32)
        lib().or_gpt_get_moment(self.h, i, which, _fp(out))
        return out

    def set_moment(self, i, which, values):
        v = f32(values).ravel()
        assert v.size == lib().or_gpt_param_len(self.h, i)
        lib().or_gpt_set_moment(self.h, i, which, _fp(v))

    def loss_and_grads(self, x, y, want_logits=False):
        x = np.ascontiguousarray(x, np.int32)
        y = np.ascontiguousarray(y, np.int32)
        logits = np.empty((x.size, self.cfg["V"]), np.float32) if want_logits else None
        loss = lib().or_gpt_loss_and_grads(self.h, x.ctypes.data_as(_i32p), y.ctypes.data_as(_i32p),
                                           _fp(logits) if want_logits else None)
        return (np.float32(loss), logits) if want_logits else np.float32(loss)

    def step(self, x, y, t):
        x = np.ascontiguousarray(x, np.int32)
        y = np.ascontiguousarray(y, np.int32)
        return np.float32(lib().or_gpt_step(self.h, x.ctypes.data_as(_i32p), y.ctypes.data_as(_i32p), t))


def set_threads(n: int):
    lib().or_set_threads(int(n))
