"""GPU tests of the HIP emitter: kernels written in the malus kernel language
(tests/emit_programs.py), lowered by malus_compile_kernels, compiled by
malus_runtime_init's hipRTC path and launched through kernel_dispatch /
kernel_dispatch_v2 at the reference's launch shapes (grid = [n] with
tg = [1] for element kernels, tg = [row length] for row kernels), against
the oracle or exact numpy.  Also the program-level gradient check of
examples/gradient_check.ml: finite differences through the emitted
perturbation kernel against the tape's gradients, gated at 1e-3 as the
reference gates it (metal_integration.rs:1141-1151)."""
import ctypes as C
import struct

import numpy as np
import pytest

import malus_amd as M
from oracle import oracle as O
from tests.emit_programs import BUILTINS, PROGRAM, SIGMOID_BACKWARD
from tests.helpers import assert_bitexact, assert_normwise, assert_ulp

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(77)


@pytest.fixture(scope="module")
def kid(rt):
    """The test programs and every builtin, emitted without builtin tags so
    each one runs its emitted HIP (not the hand-written override)."""
    reg = M.compile_kernels(PROGRAM + SIGMOID_BACKWARD, BUILTINS)
    rt.L.malus_runtime_init(*reg.init_args())
    for name, i in reg.ids.items():
        assert not rt.L.malus_kernel_is_builtin(i), name
    return reg.ids


def v1(rt, kid, name, hs):
    return rt.L.kernel_dispatch(kid[name], M.handles(hs), len(hs))


def v2(rt, kid, name, hs, grid, tg, out_shape=(), dtype=-1, uniforms=b""):
    return rt.L.kernel_dispatch_v2(kid[name], M.handles(hs), len(hs), M.sizes(grid), M.sizes(tg),
                                   M.sizes(out_shape) if out_shape else None, len(out_shape),
                                   dtype if out_shape else -1, uniforms or None, len(uniforms))


def u(fmt, *vals):
    return struct.pack("<" + fmt, *vals)


def take(rt, h):
    assert h, rt.last_error()
    out = rt.numpy(h)
    rt.free(h)
    return out


def test_emitted_builtins_match_oracle(rt, kid):
    n = 1001
    a = RNG.uniform(0.5, 2.0, n).astype(np.float32)
    b = RNG.uniform(-2.0, 2.0, n).astype(np.float32)
    s = np.float32(0.375)
    ha, hb, hs = rt.tensor(a), rt.tensor(b), rt.tensor(np.array([s], np.float32))
    for name, op in [("malus_add", O.ADD), ("malus_sub", O.SUB), ("malus_mul", O.MUL), ("malus_div", O.DIV)]:
        assert_bitexact(take(rt, v1(rt, kid, name, [ha, hb])), O.broadcast(op, a, b), name)
    for name, op, right in [("malus_add_scalar", O.ADD, True), ("malus_sub_scalar", O.SUB, True),
                            ("malus_rsub_scalar", O.SUB, False), ("malus_mul_scalar", O.MUL, True),
                            ("malus_div_scalar", O.DIV, True), ("malus_rdiv_scalar", O.DIV, False)]:
        assert_bitexact(take(rt, v1(rt, kid, name, [ha, hs])), O.scalar_op(op, a, s, right), name)
    hbb = rt.tensor(b)
    for name, op, exact in [("relu", O.RELU, True), ("abs", O.ABS, True), ("sqrt", O.SQRT, True),
                            ("exp", O.EXP, False), ("log", O.LOG, False), ("tanh", O.TANH, False),
                            ("sigmoid", O.SIGMOID, False)]:
        x, hx = (a, ha) if name in ("log", "sqrt") else (b, hbb)
        got = take(rt, v1(rt, kid, name, [hx]))
        want = O.unary(op, x)
        if exact:
            assert_bitexact(got, want, name)
        else:  # both correctly rounded from double: at most the double-rounding tie
            assert_ulp(got, want, 1, name)
    rt.free(ha, hb, hs, hbb)


def test_emitted_implicit_maps(rt, kid):
    n = 4097
    g, s = RNG.uniform(-1, 1, n).astype(np.float32), RNG.uniform(0, 1, n).astype(np.float32)
    hg, hs = rt.tensor(g), rt.tensor(s)
    assert_bitexact(take(rt, v1(rt, kid, "sigmoid_backward", [hg, hs])), (g * s) * (np.float32(1) - s), "xor kernel")
    assert_bitexact(take(rt, v1(rt, kid, "axpb", [hg, hs])), ((g + g) * s) - (-g), "axpb")
    rt.free(hg, hs)


@pytest.mark.parametrize("rows,cols", [(37, 256), (5, 1024), (64, 64)])
def test_emitted_row_softmax(rt, kid, rows, cols):
    x = (2 * RNG.standard_normal((rows, cols))).astype(np.float32)
    hx = rt.tensor(x)
    got = take(rt, v2(rt, kid, "row_softmax", [hx], [rows, 1, 1], [cols, 1, 1], uniforms=u("i", cols)))
    assert_normwise(got, O.softmax(x, 1), 1e-5, "row_softmax")
    rt.free(hx)


@pytest.mark.parametrize("sa,sb", [((6, 5, 7), (5, 1)), ((4, 8, 16), (1, 8, 1)), ((33, 65), (65,)),
                                   ((2, 3, 4, 5), (1, 1)), ((7, 9), (7, 9))])
def test_emitted_broadcast_strides_shape_ndim(rt, kid, sa, sb):
    a, b = RNG.uniform(-1, 1, sa).astype(np.float32), RNG.uniform(-1, 1, sb).astype(np.float32)
    ha, hb = rt.tensor(a), rt.tensor(b)
    got = take(rt, v2(rt, kid, "bcast_sub", [ha, hb], [a.size, 1, 1], [1, 1, 1]))
    assert_bitexact(got, a - b, f"bcast_sub {sa} {sb}")
    rt.free(ha, hb)


def test_emitted_multi_index_transpose(rt, kid):
    x = RNG.uniform(-1, 1, (37, 53)).astype(np.float32)
    hx = rt.tensor(x)
    got = take(rt, v2(rt, kid, "transpose2", [hx], [x.size, 1, 1], [1, 1, 1], out_shape=(53, 37), dtype=0))
    assert_bitexact(got, np.ascontiguousarray(x.T), "transpose2")
    rt.free(hx)


def test_emitted_gather_with_i32_indices(rt, kid):
    table = RNG.uniform(-1, 1, (65, 48)).astype(np.float32)
    idx = RNG.integers(0, 65, 300).astype(np.int32)
    idx[[3, 99, 250]] = [-1, 65, 1000]
    ht, hi = rt.tensor(table), rt.tensor(idx)
    got = take(rt, v2(rt, kid, "gather_rows", [ht, hi], [300 * 48, 1, 1], [1, 1, 1], out_shape=(300, 48), dtype=0,
                      uniforms=u("ii", 48, 65)))
    want = np.where(((idx >= 0) & (idx < 65))[:, None], table[np.clip(idx, 0, 64)], 0).astype(np.float32)
    assert_bitexact(got, want, "gather_rows")
    rt.free(ht, hi)


def test_emitted_column_sum_sequential(rt, kid):
    x = RNG.uniform(-1, 1, (3000, 96)).astype(np.float32)
    hx = rt.tensor(x)
    got = take(rt, v2(rt, kid, "col_sum", [hx], [96, 1, 1], [1, 1, 1], out_shape=(96,), dtype=0,
                      uniforms=u("i", 3000)))
    assert_bitexact(got, O.reduce_axis(O.R_SUM, x, 0), "col_sum (rows in order, as the oracle sums)")
    rt.free(hx)


def test_emitted_i32_output_argmax(rt, kid):
    x = np.round(RNG.uniform(-3, 3, (500, 65)) * 2).astype(np.float32) / 2  # ties: first index wins
    hx = rt.tensor(x)
    got = take(rt, v2(rt, kid, "row_argmax", [hx], [500, 1, 1], [1, 1, 1], out_shape=(500,), dtype=M.I32,
                      uniforms=u("i", 65)))
    assert got.dtype == np.int32
    np.testing.assert_array_equal(got, np.argmax(x, axis=1).astype(np.int32))
    rt.free(hx)


def _math_mix_ref(x, y, k):
    """math_mix with every f32 operation rounded as on the device and each
    math builtin evaluated in double and rounded once."""
    f, d = np.float32, np.float64
    r1 = lambda v: v.astype(np.float32)  # noqa: E731
    a, b, k = x, y, f(k)
    sig = f(1) / (f(1) + r1(np.exp(-b.astype(d))))
    r = (r1(np.tanh(a.astype(d))) * k + sig) - np.maximum(f(0), -a)
    den = np.maximum(np.sqrt(np.abs(a)) + f(1), r1(1.0 / np.sqrt((b * b + f(1)).astype(d))))
    r = (r + r1(np.power(np.abs(b).astype(d), 1.5))) + np.minimum(a, b) / den
    c1 = ~(a > 0) & (b < 0)
    c2 = ~c1 & ((a > b) | (b == 0))
    r = np.where(c1, r + r1(np.log((f(1) + a * a).astype(d))), r)
    r = np.where(c2, r - r1(np.exp((-a * b).astype(d))), r)
    return r.astype(np.float32)


def test_emitted_math_builtins_pow_and_logic(rt, kid):
    n = 4096
    x = RNG.uniform(-2, 2, n).astype(np.float32)
    y = RNG.uniform(-2, 2, n).astype(np.float32)
    y[:64] = 0.0
    hx, hy = rt.tensor(x), rt.tensor(y)
    got = take(rt, v2(rt, kid, "math_mix", [hx, hy], [n, 1, 1], [1, 1, 1], uniforms=u("f", 0.75)))
    assert_normwise(got, _math_mix_ref(x, y, 0.75), 1e-6, "math_mix")
    rt.free(hx, hy)


def test_emitted_kernel_abi_checks(rt, kid):
    x = RNG.uniform(-1, 1, 64).astype(np.float32)
    hx, hshort = rt.tensor(x), rt.tensor(x[:10])
    reg = M.compile_kernels("kernel widen(a: Tensor<i64>, b: Tensor<f32>) -> Tensor<f32>:\n    return b\n")
    rt.L.malus_runtime_init(*reg.init_args())
    wid = reg.ids["widen"]
    rt.L.malus_set_abort_on_error(0)
    try:
        # the uniforms blob must be the size the emitted kernel declares
        assert v2(rt, kid, "nudge", [hx], [64, 1, 1], [1, 1, 1], uniforms=u("i", 3)) == 0
        assert "takes 8 bytes of uniforms" in rt.last_error()
        rt.L.malus_clear_error()
        # an implicit map reads every input at each output index
        assert v1(rt, kid, "malus_add", [hx, hshort]) == 0
        assert "shorter than" in rt.last_error()
        rt.L.malus_clear_error()
        # the element widths the kernel declares must be the tensors' (the
        # output takes input 0's dtype, metal.rs:1878-1888)
        h64 = rt.tensor(np.arange(64, dtype=np.int64))
        assert v1(rt, kid, "malus_add", [h64, hx]) == 0
        assert "writes 4-byte elements" in rt.last_error()
        rt.L.malus_clear_error()
        assert rt.L.kernel_dispatch(wid, M.handles([h64, hx]), 2) == 0
        assert "writes 4-byte elements, but its output takes input 0's dtype (8-byte elements)" in rt.last_error()
        rt.L.malus_clear_error()
        assert rt.L.kernel_dispatch(wid, M.handles([hx, hx]), 2) == 0
        assert "reads input 0 as 8-byte elements" in rt.last_error()
        rt.L.malus_clear_error()
        rt.free(h64)
    finally:
        rt.L.malus_set_abort_on_error(1)
    rt.free(hx, hshort)


# ------------------------------------------------- program-level gradient check
OP = dict(Matmul=0, Add=1, Mul=3, Sum=12, Softmax=20, Layernorm=21, Gelu=22, CrossEntropy=23, Embedding=24)


class GradCheck:
    """examples/gradient_check.ml's procedure through the C ABI: analytic
    gradients from the tape; numeric ones from central differences of the
    loss at inputs moved by the emitted perturbation kernel
    (`nudge`, the __perturb_fwd launch: grid=[n], tg=[1]); every
    |analytic - numeric| goes to malus_record_diff."""

    def __init__(self, rt, kid):
        self.rt, self.kid = rt, kid

    def nudge(self, h, i, delta):
        n = self.rt.L.tensor_len(h)
        out = v2(self.rt, self.kid, "nudge", [h], [n, 1, 1], [1, 1, 1], uniforms=u("if", i, delta))
        assert out, self.rt.last_error()
        return out

    def run(self, inputs, loss_fn, eps):
        rt = self.rt
        L = rt.L
        L.tape_reset()
        for h in inputs:
            L.tape_register_leaf(h)
        loss = loss_fn(inputs, True)
        L.backward(loss)
        grads = []
        for h in inputs:
            g = L.tape_get_grad(h)
            grads.append(rt.numpy(g).ravel())
            rt.free(g)
        rt.free(loss)
        L.tape_reset()
        for k, h in enumerate(inputs):
            for i in range(L.tensor_len(h)):
                vals = []
                for delta in (eps, -eps):
                    hp = self.nudge(h, i, delta)
                    args = list(inputs)
                    args[k] = hp
                    lh = loss_fn(args, False)
                    vals.append(L.malus_tensor_get_f32(lh, 0))
                    rt.free(hp, lh)
                numeric = (vals[0] - vals[1]) / (2.0 * eps)
                L.malus_record_diff(abs(numeric - float(grads[k][i])))


def _wsum(rt, out, w, record):
    """sum(out * w) with the tape records the JIT would make."""
    L = rt.L
    prod = L.malus_std_broadcast_fwd(M.MUL, out, w)
    if record:
        L.tape_record_binop(OP["Mul"], out, w, prod)
    s = L.malus_std_reduce_all_sum_fwd(prod)
    if record:
        L.tape_record_unary(OP["Sum"], prod, s)
    return s


def test_gradient_check_program_with_emitted_perturbation(rt, kid):
    L = rt.L
    gc = GradCheck(rt, kid)
    L.malus_gradcheck_reset()

    def t(*vals, shape=None):
        a = np.array(vals, np.float32)
        return rt.tensor(a.reshape(shape) if shape else a)

    w4 = t(0.3, -0.2, 0.25, 0.1, -0.15, 0.4, 0.2, -0.35, shape=(2, 4))

    def add(ins, rec):
        o = L.malus_std_broadcast_fwd(M.ADD, ins[0], ins[1])
        if rec:
            L.tape_record_binop(OP["Add"], ins[0], ins[1], o)
        s = L.malus_std_reduce_all_sum_fwd(o)
        if rec:
            L.tape_record_unary(OP["Sum"], o, s)
        return s

    def mul(ins, rec):
        o = L.malus_std_broadcast_fwd(M.MUL, ins[0], ins[1])
        if rec:
            L.tape_record_binop(OP["Mul"], ins[0], ins[1], o)
        s = L.malus_std_reduce_all_sum_fwd(o)
        if rec:
            L.tape_record_unary(OP["Sum"], o, s)
        return s

    def matmul(ins, rec):
        o = L.tensor_matmul(ins[0], ins[1])
        if rec:
            L.tape_record_binop(OP["Matmul"], ins[0], ins[1], o)
        s = L.malus_std_reduce_all_sum_fwd(o)
        if rec:
            L.tape_record_unary(OP["Sum"], o, s)
        return s

    def softmax(ins, rec):
        o = L.malus_std_softmax_fwd(ins[0], 1)
        if rec:
            L.tape_record_reduce(OP["Softmax"], ins[0], o, 1, 0)
        s = _wsum(rt, o, w4, rec)
        if not rec:
            rt.free(o)
        return s

    def layernorm(ins, rec):
        var = C.c_int64()
        o = L.malus_std_layernorm_fwd(ins[0], 1, C.byref(var))
        if rec:
            L.tape_record_layernorm(OP["Layernorm"], ins[0], o, var.value, 1)
        else:
            rt.free(var.value)
        return _wsum(rt, o, w4, rec)

    def gelu(ins, rec):
        o = L.malus_std_gelu_fwd(ins[0])
        if rec:
            L.tape_record_unary(OP["Gelu"], ins[0], o)
        return _wsum(rt, o, w4, rec)

    tg = rt.tensor(np.array([2, 0], np.int32))

    def cross_entropy(ins, rec):
        probs = C.c_int64()
        o = L.malus_std_cross_entropy_fwd(ins[0], tg, C.byref(probs))
        if rec:
            L.tape_record_cross_entropy(OP["CrossEntropy"], ins[0], o, probs.value, tg)
        else:
            rt.free(probs.value)
        return o

    idx = rt.tensor(np.array([0, 3, 3, 1], np.int32))
    we = t(*RNG.uniform(-1, 1, 12), shape=(4, 3))

    def embedding(ins, rec):
        o = L.malus_std_embedding_fwd(ins[0], idx)
        if rec:
            L.tape_record_embedding(OP["Embedding"], ins[0], idx, o)
        return _wsum(rt, o, we, rec)

    x3, y3 = t(1.0, 2.0, 3.0), t(0.5, -1.0, 2.0)
    gc.run([x3, y3], add, 1e-3)
    gc.run([x3, y3], mul, 1e-3)
    gc.run([t(1, 2, 3, 4, shape=(2, 2)), t(0.5, -0.5, 1, 2, shape=(2, 2))], matmul, 1e-2)  # linear: the larger eps
    xs = t(1.0, 2.0, 3.0, 4.0, 0.5, 1.5, -0.5, 2.5, shape=(2, 4))
    gc.run([xs], softmax, 1e-3)
    gc.run([t(1.0, 2.0, 3.5, 4.0, 0.5, -1.5, -0.5, 2.5, shape=(2, 4))], layernorm, 1e-3)
    gc.run([t(1.0, -1.0, 0.0, 2.0, -2.0, 0.5, -0.5, 3.0, shape=(2, 4))], gelu, 1e-3)
    gc.run([t(0.2, -0.3, 0.9, 0.1, 1.0, -0.5, 0.3, 0.4, shape=(2, 4))], cross_entropy, 1e-3)
    gc.run([t(*RNG.uniform(-1, 1, 12), shape=(4, 3))], embedding, 1e-3)
    worst = L.malus_gradcheck_max_diff()
    assert worst < 1e-3, f"max |analytic - numeric| = {worst}"
    L.tape_reset()
    rt.free(w4, tg, idx, we, x3, y3, xs)
