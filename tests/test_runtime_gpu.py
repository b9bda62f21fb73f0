"""GPU tests of the runtime ABI: handles, pool, pending/flush, printing, the
tape (known answers of crates/malus-runtime/src/tests.rs), the
kernel_dispatch / kernel_dispatch_v2 override path a JIT'd program uses, and
hipRTC-compiled user kernels."""
import ctypes as C
import struct

import numpy as np
import pytest

import malus_amd as M
from oracle import oracle as O
from tests.helpers import KATS, assert_bitexact, assert_normwise

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(99)
OP = dict(Matmul=0, Add=1, Sub=2, Mul=3, Div=4, Sigmoid=5, Relu=6, Tanh=7, Exp=8, Log=9, Sqrt=10, Abs=11, Sum=12,
          Transpose=13, Neg=14, ReduceSumAxis=15, Reshape=19, Softmax=20, Layernorm=21, Gelu=22, CrossEntropy=23,
          Embedding=24)


def f32(*v):
    return np.array(v, np.float32)


# --------------------------------------------------------------- handles
def test_alloc_roundtrip_and_metadata(rt):
    a = RNG.standard_normal((3, 4, 5)).astype(np.float32)
    h = rt.tensor(a)
    assert rt.L.tensor_len(h) == 60 and rt.L.tensor_ndim(h) == 3
    assert rt.L.tensor_dim(h, -1) == 5 and rt.L.tensor_dim(h, 0) == 3
    assert_bitexact(rt.numpy(h), a)
    assert rt.L.malus_tensor_get_f32(h, 7) == a.ravel()[7]
    for dt in (np.int32, np.int64):
        hi = rt.tensor(np.arange(10, dtype=dt))
        assert rt.numpy(hi).tolist() == list(range(10))
        rt.free(hi)
    rt.free(h)


def test_zeros_ones_null_and_empty(rt):
    hz = rt.L.tensor_alloc_zeros_gpu(M.sizes([4, 5]), 2)
    ho = rt.L.tensor_alloc_ones_gpu(M.sizes([7]), 1)
    assert np.all(rt.numpy(hz) == 0) and np.all(rt.numpy(ho) == 1)
    hn = rt.L.tensor_alloc_gpu(0, M.sizes([16]), 1, None)  # null data: contents unspecified
    he = rt.L.tensor_alloc_zeros_gpu(M.sizes([0]), 1)
    assert rt.L.tensor_len(he) == 0
    rt.free(hz, ho, hn, he)


def test_retain_release_and_rc_counters(rt):
    rt.L.malus_rc_reset()
    h = rt.tensor(f32(1, 2, 3))
    rt.L.tensor_retain(h)
    rt.L.tensor_release(h)
    assert rt.numpy(h).tolist() == [1, 2, 3]  # still alive
    rt.L.tensor_release(h)
    c = (C.c_int64 * 3)()
    rt.L.malus_rc_counts(c)
    assert c[0] == 1 and c[1] == 2 and c[2] == 1
    rt.L.tensor_retain(0)
    rt.L.tensor_release(0)  # null handles are no-ops


def test_pool_reuses_freed_buffers(rt):
    st = (C.c_int64 * 4)()
    h = rt.L.tensor_alloc_zeros_gpu(M.sizes([12345]), 1)
    rt.free(h)
    rt.L.malus_pool_stats(st)
    hits0 = st[0]
    h = rt.L.tensor_alloc_zeros_gpu(M.sizes([12345]), 1)
    rt.L.malus_pool_stats(st)
    assert st[0] == hits0 + 1
    assert np.all(rt.numpy(h) == 0)  # pooled buffers are re-zeroed
    rt.free(h)


def test_pending_then_flush_on_read(rt):
    a = rt.tensor(RNG.standard_normal((512, 512)).astype(np.float32))
    c = rt.L.tensor_matmul(a, a)
    d = rt.L.tensor_matmul(c, a)
    r = rt.L.tensor_reshape(d, M.sizes([512 * 512]), 1)
    assert rt.L.tensor_is_pending(r) == rt.L.tensor_is_pending(d)  # alias inherits pending state
    _ = rt.L.malus_tensor_get_f32(r, 0)
    assert rt.L.tensor_is_pending(d) == 0 and rt.L.tensor_is_pending(r) == 0
    rt.free(a, c, d, r)


def test_reshape_alias_and_count_mismatch(rt):
    h = rt.tensor(np.arange(6, dtype=np.float32))
    r = rt.L.tensor_reshape(h, M.sizes([2, 3]), 2)
    assert rt.shape(r) == (2, 3) and rt.numpy(r).ravel().tolist() == list(range(6))
    rt.free(h)  # the alias keeps the storage alive
    assert rt.numpy(r).ravel().tolist() == list(range(6))
    rt.L.malus_set_abort_on_error(0)
    try:
        bad = rt.L.tensor_reshape(r, M.sizes([4, 2]), 2)
        assert bad == 0 and "reshape element count mismatch" in rt.last_error()
    finally:
        rt.L.malus_set_abort_on_error(1)
    rt.free(r)


def test_matmul_shape_error_message(rt):
    a, b = rt.tensor(np.ones((2, 3), np.float32)), rt.tensor(np.ones((4, 2), np.float32))
    rt.L.malus_set_abort_on_error(0)
    try:
        assert rt.L.tensor_matmul(a, b) == 0
        assert "matmul shape mismatch" in rt.last_error() and "[2x3] @ [4x2]" in rt.last_error()
    finally:
        rt.L.malus_set_abort_on_error(1)
    rt.free(a, b)


def test_device_side_index_check(rt):
    w = rt.tensor(np.ones((4, 8), np.float32))
    idx = rt.tensor(np.array([0, 9, 1], np.int32))
    rt.L.malus_set_abort_on_error(0)
    try:
        out = rt.L.malus_std_embedding_fwd(w, idx)
        rt.L.gpu_barrier()
        assert "embedding index out of range" in rt.last_error()
        rt.L.malus_clear_error()
        rt.L.gpu_barrier()  # the flag is cleared once reported
        assert rt.last_error() == ""
    finally:
        rt.L.malus_set_abort_on_error(1)
    rt.free(w, idx, out)


def test_print_formats_like_rust_display(rt, capfd):
    h = rt.tensor(np.array([[0.5, 1.0, -1e9], [0.1, 0.0056860363, 3.0]], np.float32))
    rt.L.tensor_print(h)
    out = capfd.readouterr().out
    assert out == "[[0.5, 1, -1000000000], [0.1, 0.0056860363, 3]]"
    hi = rt.tensor(np.array([[1, -2], [3, 4]], np.int32))
    rt.L.tensor_print(hi)
    assert capfd.readouterr().out == "[[1, -2], [3, 4]]"
    rt.free(h, hi)


def test_randn_uniform_int_match_oracle(rt):
    rt.L.malus_rng_set_counter(5)
    h = rt.L.tensor_randn(M.sizes([3, 7]), 2)
    assert_bitexact(rt.numpy(h), O.randn(5, (3, 7)), "randn")
    u = rt.L.malus_rand_uniform()
    assert u == O.lib().or_rand_uniform(6)
    assert rt.L.malus_rand_int(65) == O.lib().or_rand_int(7, 65)
    assert rt.L.malus_rng_get_counter() == 8
    rt.free(h)


def test_buffer_freeze(rt):
    b = rt.L.malus_buffer_i32(5)
    for i in range(5):
        rt.L.malus_buffer_set_i32(b, i, 10 * i)
    assert rt.L.malus_buffer_get_i32(b, 3) == 30
    h = rt.L.malus_buffer_freeze_i32(b)
    assert rt.L.malus_tensor_dtype(h) == 5 and rt.numpy(h).tolist() == [0, 10, 20, 30, 40]
    rt.L.malus_buffer_free(b)
    rt.free(h)


def test_causal_mask_bitexact(rt):
    h = rt.L.tensor_causal_mask(65)
    assert_bitexact(rt.numpy(h), O.causal_mask(65), "mask")
    rt.free(h)


def test_bench_warm_median(rt):
    # bench.rs:51-70: skip 3 warmup steps; even count -> mean of the middle two
    rt.L.bench_reset()
    for ms in (100, 100, 100, 4, 2, 3, 1):
        rt.L.malus_bench_record(ms)
    med, mn, mx, n = C.c_double(), C.c_double(), C.c_double(), C.c_int64()
    assert rt.L.bench_report(C.byref(med), C.byref(mn), C.byref(mx), C.byref(n)) == 1
    assert (med.value, mn.value, mx.value, n.value) == (2.5, 1, 4, 4)
    rt.L.bench_reset()


# ------------------------------------------------------------------ tape
def leaf(rt, *vals):
    h = rt.tensor(f32(*vals))
    rt.L.tape_register_leaf(h)
    return h


def grad(rt, h):
    g = rt.L.tape_get_grad(h)
    out = rt.numpy(g)
    rt.free(g)
    return out


@pytest.fixture
def tape(rt):
    rt.L.tape_reset()
    yield rt
    rt.L.tape_reset()


@pytest.mark.parametrize("kat", KATS["backward_binop"], ids=lambda k: k["op"])
def test_backward_binop_kats(tape, kat):
    rt = tape
    op, a, b, ga, gb = kat["op"], kat["a"], kat["b"], kat["ga"], kat["gb"]
    ha, hb = leaf(rt, *a), leaf(rt, *b)
    out = rt.L.malus_std_broadcast_fwd(OP[op] - 1, ha, hb)
    rt.L.tape_record_binop(OP[op], ha, hb, out)
    rt.L.backward(out)
    np.testing.assert_allclose(grad(rt, ha), ga, atol=1e-6)
    np.testing.assert_allclose(grad(rt, hb), gb, atol=1e-6)
    rt.free(ha, hb, out)


UNARY_FN = {"Relu": M.RELU, "Sigmoid": M.SIGMOID, "Tanh": M.TANH, "Exp": M.EXP, "Log": M.LOG, "Sqrt": M.SQRT,
            "Abs": M.ABS}


@pytest.mark.parametrize("kat", [k for k in KATS["backward_unary"] if k["op"] in UNARY_FN], ids=lambda k: k["op"])
def test_backward_unary_kats(tape, kat):
    rt = tape
    op, x, want = kat["op"], kat["x"], kat["gx"]
    hx = leaf(rt, *x)
    out = rt.L.malus_std_unary(UNARY_FN[op], hx)
    rt.L.tape_record_unary(OP[op], hx, out)
    rt.L.backward(out)
    np.testing.assert_allclose(grad(rt, hx), want, atol=1e-6)
    rt.free(hx, out)


def test_backward_neg_sum_transpose_matmul(tape):
    rt = tape
    a = leaf(rt, 1, -2, 3)
    out = rt.L.malus_std_scalar_op(M.MUL, a, -1.0, 0)
    rt.L.tape_record_unary(OP["Neg"], a, out)
    rt.L.backward(out)
    assert grad(rt, a).tolist() == [-1, -1, -1]
    s = rt.L.malus_std_reduce_all_sum_fwd(a)
    rt.L.tape_zero_grad(M.handles([a]), 1)
    rt.L.tape_record_unary(OP["Sum"], a, s)
    rt.L.backward(s)
    assert grad(rt, a).tolist() == [1, 1, 1]
    rt.free(out, s, a)
    # tests.rs:749-780: ones[2,2] seed, dA = ones @ B^T -> [3, 7, 11]
    A = rt.tensor(np.array([[1, 0, 0], [1, 0, 0]], np.float32))
    B = rt.tensor(np.array([[1, 2], [3, 4], [5, 6]], np.float32))
    rt.L.tape_register_leaf(A)
    rt.L.tape_register_leaf(B)
    Cm = rt.L.tensor_matmul(A, B)
    rt.L.tape_record_binop(OP["Matmul"], A, B, Cm)
    rt.L.backward(Cm)
    assert grad(rt, A)[0].tolist() == [3, 7, 11]
    assert grad(rt, B).shape == (3, 2)
    T = rt.tensor(np.array([[1, 2], [3, 4]], np.float32))
    rt.L.tape_register_leaf(T)
    TT = rt.L.tensor_permute(T, None, 0)
    rt.L.tape_record_perm(OP["Transpose"], T, TT, None, 0)
    rt.L.backward(TT)
    assert grad(rt, T).tolist() == [[1, 1], [1, 1]]
    rt.free(A, B, Cm, T, TT)


def test_matmul_vjps_with_both_operands_watched(tape):
    """A @ B with both operands watched (dA and dB from the two VJP GEMMs),
    then X @ X, whose two VJPs add into the one gradient.  Gradients against
    float64 products of the same inputs."""
    rt = tape
    rng = np.random.default_rng(11)
    av = rng.uniform(-1, 1, (300, 200)).astype(np.float32)
    bv = rng.uniform(-1, 1, (200, 96)).astype(np.float32)
    xv = rng.uniform(-1, 1, (96, 96)).astype(np.float32)
    A, B, X = rt.tensor(av), rt.tensor(bv), rt.tensor(xv)
    for h in (A, B, X):
        rt.L.tape_register_leaf(h)
    Cm = rt.L.tensor_matmul(A, B)
    rt.L.tape_record_binop(OP["Matmul"], A, B, Cm)
    rt.L.backward(Cm)
    ones = np.ones((300, 96))
    np.testing.assert_allclose(grad(rt, A), ones @ bv.T.astype(np.float64), rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(grad(rt, B), av.T.astype(np.float64) @ ones, rtol=1e-5, atol=1e-4)
    Xm = rt.L.tensor_matmul(X, X)
    rt.L.tape_record_binop(OP["Matmul"], X, X, Xm)
    rt.L.backward(Xm)
    o2 = np.ones((96, 96))
    want = o2 @ xv.T.astype(np.float64) + xv.T.astype(np.float64) @ o2
    np.testing.assert_allclose(grad(rt, X), want, rtol=1e-5, atol=1e-4)
    rt.free(A, B, X, Cm, Xm)


def test_grad_accumulates_across_backwards_and_zero_grad(tape):
    rt = tape
    a = leaf(rt, 2)
    for bval in (3, 7):
        b = rt.tensor(f32(bval))
        out = rt.L.malus_std_broadcast_fwd(M.ADD, a, b)
        rt.L.tape_record_binop(OP["Add"], a, b, out)
        rt.L.backward(out)
        rt.free(b, out)
    assert grad(rt, a).tolist() == [2.0]
    rt.L.tape_zero_grad(M.handles([a]), 1)
    assert grad(rt, a).tolist() == [0.0]
    lens = (C.c_size_t * 2)()
    rt.L.malus_tape_registry_lens(lens)
    assert lens[0] == 1
    rt.free(a)
    rt.L.malus_tape_registry_lens(lens)
    assert lens[0] == 0 and lens[1] == 0  # releasing a leaf drops its registry entries


def test_released_leaf_gradient_is_not_computed(tape):
    # out = x * s with s a [1] leaf.  While the program holds s, backward
    # computes ds = sum(dout * x) (tape.rs:460-469 computes both VJPs); once
    # the program has released s (only the tape still references it, so its
    # grad can never be queried) that VJP is skipped.  dx is the same either way.
    rt = tape
    xv = np.random.default_rng(5).uniform(-1, 1, (64, 32)).astype(np.float32)

    def step(keep_s):
        x = leaf(rt, *xv.ravel())
        s = leaf(rt, 0.5)
        out = rt.L.malus_std_broadcast_fwd(M.MUL, x, s)
        rt.L.tape_record_binop(OP["Mul"], x, s, out)
        if not keep_s:
            rt.free(s)
        rt.L.malus_rc_reset()
        rt.L.backward(out)
        c = (C.c_int64 * 3)()
        rt.L.malus_rc_counts(c)
        gx = grad(rt, x)
        gs = grad(rt, s) if keep_s else None
        rt.free(x, out, *([s] if keep_s else []))
        rt.L.tape_reset()
        return c[2], gx, gs

    allocs_live, gx_live, gs = step(True)
    allocs_dead, gx_dead, _ = step(False)
    np.testing.assert_allclose(gs, [xv.astype(np.float64).sum()], rtol=1e-5, atol=1e-3)
    assert_bitexact(gx_dead, gx_live, "dx")
    assert np.all(gx_live == 0.5)
    assert allocs_dead < allocs_live, (allocs_dead, allocs_live)


def test_broadcast_add_backward_reduces_to_operand_shape(tape):
    # tests.rs:1130-1177: (1,3) + (2,3), loss = sum -> da = [[2,2,2]], db = ones
    rt = tape
    a = rt.tensor(np.ones((1, 3), np.float32))
    b = rt.tensor(np.ones((2, 3), np.float32))
    rt.L.tape_register_leaf(a)
    rt.L.tape_register_leaf(b)
    out = rt.L.malus_std_broadcast_fwd(M.ADD, a, b)
    rt.L.tape_record_binop(OP["Add"], a, b, out)
    s = rt.L.malus_std_reduce_all_sum_fwd(out)
    rt.L.tape_record_unary(OP["Sum"], out, s)
    rt.L.backward(s)
    ga, gb = grad(rt, a), grad(rt, b)
    assert ga.shape == (1, 3) and np.all(ga == 2)
    assert gb.shape == (2, 3) and np.all(gb == 1)
    rt.free(a, b, out, s)


def test_reshape_and_reduce_vjps(tape):
    rt = tape
    x = rt.tensor(np.arange(6, dtype=np.float32).reshape(2, 3))
    rt.L.tape_register_leaf(x)
    r = rt.L.tensor_reshape(x, M.sizes([3, 2]), 2)
    rt.L.tape_record_unary(OP["Reshape"], x, r)
    s = rt.L.malus_std_reduce_fwd(M.R_SUM, r, 0, 0)
    rt.L.tape_record_reduce(OP["ReduceSumAxis"], r, s, 0, 0)
    rt.L.backward(s)
    g = grad(rt, x)
    assert g.shape == (2, 3) and np.all(g == 1)
    rt.free(x, r, s)


# --------------------------------------------- kernel_dispatch(_v2): JIT path
BUILTINS = ["__broadcast_add_kernel", "__broadcast_sub_kernel", "__broadcast_mul_kernel", "__broadcast_div_kernel",
            "__reduce_sum_kernel", "__reduce_mean_kernel", "__reduce_max_kernel", "__reduce_var_kernel",
            "__softmax_kernel", "__layernorm_kernel", "__layernorm_var_kernel", "__gelu_kernel",
            "__cross_entropy_nll_kernel", "__embedding_kernel", "__transpose_2d_kernel", "__permute_3d_kernel",
            "__permute_nd_kernel", "__scale_kernel", "__fill_like_kernel", "__eq_kernel", "__sigmoid_bwd_kernel",
            "__relu_bwd_kernel", "__tanh_bwd_kernel", "__sqrt_bwd_kernel", "__abs_bwd_kernel",
            "__expand_axis_kernel", "__rsqrt_eps_kernel", "__gelu_bwd_kernel", "__cross_entropy_bwd_kernel",
            "__embedding_bwd_kernel", "malus_add", "malus_sub", "malus_mul", "malus_div", "malus_add_scalar",
            "malus_sub_scalar", "malus_mul_scalar", "malus_div_scalar", "malus_rsub_scalar", "malus_rdiv_scalar",
            "relu", "sigmoid", "tanh", "exp", "log", "sqrt", "abs"]
BASE_ID = 1000


@pytest.fixture(scope="module")
def kid(rt):
    ids = (C.c_uint64 * len(BUILTINS))(*[BASE_ID + i for i in range(len(BUILTINS))])
    srcs = (C.c_char_p * len(BUILTINS))(*[f"//@malus-builtin {n}\n".encode() for n in BUILTINS])
    rt.L.malus_runtime_init(ids, srcs, len(BUILTINS))
    return {n: BASE_ID + i for i, n in enumerate(BUILTINS)}


def v2(rt, kid, name, hs, grid, tg, out_shape=(), dtype=-1, uniforms=b""):
    return rt.L.kernel_dispatch_v2(kid[name], M.handles(hs), len(hs), M.sizes(grid), M.sizes(tg),
                                   M.sizes(out_shape) if out_shape else None, len(out_shape),
                                   dtype if out_shape else -1, uniforms or None, len(uniforms))


def u(fmt, *vals):
    return struct.pack("<" + fmt, *vals)


def test_v2_stdlib_launch_shapes_match_host_fns(rt, kid):
    # launches exactly as the .ml host fns issue them (tg = [axis] or [1])
    x = RNG.standard_normal((65, 1536)).astype(np.float32)  # axis > 1024: the reference's cap
    hx = rt.tensor(x)
    hs = v2(rt, kid, "__softmax_kernel", [hx], [65, 1, 1], [1536, 1, 1], uniforms=u("ii", 1536, 1))
    assert_normwise(rt.numpy(hs), O.softmax(x, 1), 1e-5, "softmax via v2")
    hr = v2(rt, kid, "__reduce_sum_kernel", [hx], [1536, 1, 1], [65, 1, 1], out_shape=(1536,), dtype=0,
            uniforms=u("ii", 65, 1536))
    assert_normwise(rt.numpy(hr), O.reduce_axis(O.R_SUM, x, 0), 1e-5, "reduce axis 0 via v2")
    hl = v2(rt, kid, "__layernorm_kernel", [hx], [65, 1, 1], [1536, 1, 1], uniforms=u("iif", 1536, 1, 1e-5))
    assert_normwise(rt.numpy(hl), O.layernorm(x, 1)[0], 1e-5, "layernorm via v2")
    hv = v2(rt, kid, "__layernorm_var_kernel", [hx], [65, 1, 1], [1536, 1, 1], uniforms=u("iif", 1536, 1, 1e-5))
    var = rt.numpy(hv)
    assert var.shape == x.shape  # full-shape variance, as layernorm.ml:71 produces it
    assert_normwise(var[:, 0:1], O.layernorm(x, 1)[1], 1e-5, "var via v2")
    hb = rt.tensor(RNG.standard_normal(1536).astype(np.float32))
    hm = v2(rt, kid, "__broadcast_mul_kernel", [hx, hb], [65 * 1536, 1, 1], [1, 1, 1])
    assert_bitexact(rt.numpy(hm), O.broadcast(O.MUL, x, rt.numpy(hb)), "bcast via v2")
    ht = v2(rt, kid, "__transpose_2d_kernel", [hx], [65 * 1536, 1, 1], [1, 1, 1], out_shape=(1536, 65), dtype=0)
    assert_bitexact(rt.numpy(ht), x.T.copy(), "transpose via v2")
    he = v2(rt, kid, "__expand_axis_kernel", [hr], [65 * 1536, 1, 1], [1, 1, 1], out_shape=(65, 1536), dtype=0,
            uniforms=u("ii", 65, 1536))
    assert_bitexact(rt.numpy(he), np.broadcast_to(rt.numpy(hr), (65, 1536)), "expand via v2")
    rt.free(hx, hs, hr, hl, hv, hb, hm, ht, he)


def test_v2_index_and_vjp_kernels(rt, kid):
    w = RNG.standard_normal((65, 96)).astype(np.float32)
    idx = RNG.integers(0, 65, 300).astype(np.int32)
    hw, hi = rt.tensor(w), rt.tensor(idx)
    he = v2(rt, kid, "__embedding_kernel", [hw, hi], [300 * 96, 1, 1], [1, 1, 1], out_shape=(300, 96), dtype=0,
            uniforms=u("i", 96))
    assert_bitexact(rt.numpy(he), O.embedding(w, idx), "embedding via v2")
    hb = v2(rt, kid, "__embedding_bwd_kernel", [he, hi], [65 * 96, 1, 1], [1, 1, 1], out_shape=(65, 96), dtype=0,
            uniforms=u("ii", 300, 96))
    assert_bitexact(rt.numpy(hb), O.embedding_bwd(rt.numpy(he), idx, 65), "embedding bwd via v2")
    logits = RNG.standard_normal((300, 65)).astype(np.float32)
    probs = O.softmax(logits, 1)
    hp = rt.tensor(probs)
    hn = v2(rt, kid, "__cross_entropy_nll_kernel", [hp, hi], [300, 1, 1], [1, 1, 1], out_shape=(300,), dtype=0,
            uniforms=u("i", 65))
    from tests.helpers import assert_ulp
    want_nll = -O.unary(O.LOG, probs[np.arange(300), idx])
    assert_ulp(rt.numpy(hn), want_nll, 2, "nll via v2")
    hg = v2(rt, kid, "__cross_entropy_bwd_kernel", [hp, hi], [300 * 65, 1, 1], [1, 1, 1], uniforms=u("if", 65, 1 / 300))
    assert_bitexact(rt.numpy(hg), O.cross_entropy_bwd(probs, idx, 1.0), "ce bwd via v2")
    x4 = RNG.standard_normal((2, 3, 4, 8)).astype(np.float32)
    h4 = rt.tensor(x4)
    hp4 = v2(rt, kid, "__permute_nd_kernel", [h4], [192, 1, 1], [1, 1, 1], out_shape=(2, 4, 3, 8), dtype=0,
             uniforms=u("8i", 0, 2, 1, 3, 0, 0, 0, 0))
    assert_bitexact(rt.numpy(hp4), O.permute(x4, (0, 2, 1, 3)), "permute_nd via v2")
    rt.free(hw, hi, he, hb, hp, hn, hg, h4, hp4)


def test_v2_unary_bwd_helper_kernels(rt, kid):
    # __scale_kernel, __fill_like_kernel, __eq_kernel (unary_bwd.ml:6-34) and
    # __rsqrt_eps_kernel (transformer_bwd.ml:6-12) by tag, at the host fns'
    # launch shape grid=[n], tg=[1], with the output shaped like input 0.
    n = 70001
    x = RNG.standard_normal((7, n // 7)).astype(np.float32)
    y = np.where(RNG.random(x.shape) < 0.3, x, RNG.standard_normal(x.shape)).astype(np.float32)
    hx, hy = rt.tensor(x), rt.tensor(y)
    hs = v2(rt, kid, "__scale_kernel", [hx], [n, 1, 1], [1, 1, 1], uniforms=u("f", -0.375))
    assert rt.shape(hs) == x.shape
    assert_bitexact(rt.numpy(hs), O.scalar_op(O.MUL, x, -0.375), "scale via v2")
    hf = v2(rt, kid, "__fill_like_kernel", [hx], [n, 1, 1], [1, 1, 1], uniforms=u("f", 2.5))
    assert_bitexact(rt.numpy(hf), np.full(x.shape, 2.5, np.float32), "fill_like via v2")
    he = v2(rt, kid, "__eq_kernel", [hx, hy], [n, 1, 1], [1, 1, 1])
    eq = rt.numpy(he)
    assert_bitexact(eq, (x == y).astype(np.float32), "eq via v2")
    assert 0.2 < eq.mean() < 0.4
    v = RNG.uniform(0, 4, x.shape).astype(np.float32)
    v.flat[:3] = [0.0, 1e-30, 3.0]
    hv = rt.tensor(v)
    hr = v2(rt, kid, "__rsqrt_eps_kernel", [hv], [n, 1, 1], [1, 1, 1], uniforms=u("f", 1e-5))
    # 1/sqrt(v + eps) in f32: an IEEE add, square root and division
    want = np.float32(1) / np.sqrt(v + np.float32(1e-5))
    assert_bitexact(rt.numpy(hr), want, "rsqrt_eps via v2")
    rt.free(hx, hy, hs, hf, he, hv, hr)


def test_v1_builtins(rt, kid):
    a = RNG.uniform(0.5, 2, 1001).astype(np.float32)
    b = RNG.uniform(0.5, 2, 1001).astype(np.float32)
    ha, hb, hs = rt.tensor(a), rt.tensor(b), rt.tensor(f32(0.25))
    for name, want in [("malus_sub", a - b), ("malus_div", a / b), ("malus_rsub_scalar", np.float32(0.25) - a),
                       ("malus_div_scalar", a / np.float32(0.25)), ("relu", np.maximum(a, 0))]:
        hsec = hs if "scalar" in name else hb
        hh = M.handles([ha] if name == "relu" else [ha, hsec])
        h = rt.L.kernel_dispatch(kid[name], hh, 1 if name == "relu" else 2)
        assert_bitexact(rt.numpy(h), want.astype(np.float32), name)
        rt.free(h)
    rt.free(ha, hb, hs)


SIGMOID_BACKWARD_HIP = """
extern "C" __global__ void malus_kernel_{id}(const float* grad_out, const float* sig_z, float* out, unsigned n) {{
  unsigned tid = blockIdx.x * blockDim.x + threadIdx.x;
  if (tid >= n) return;
  out[tid] = ((grad_out[tid] * sig_z[tid]) * (1.0f - sig_z[tid]));
}}
"""

# metal_integration.rs:166-190 softmax de-risk kernel, explicit form (v2 ABI)
SOFTMAX_V2_HIP = """
struct TensorMeta {{ unsigned ndim; unsigned shape[8]; unsigned strides[8]; }};
struct Uniforms_{id} {{ int cols; }};
extern "C" __global__ void malus_kernel_{id}(const float* input, float* out, Uniforms_{id} u,
                                            TensorMeta input_meta, TensorMeta out_meta) {{
  int row = blockIdx.x, col = threadIdx.x, start = row * u.cols;
  __shared__ float scratch[1024];
  scratch[col] = input[start + col];
  __syncthreads();
  float m = scratch[0];
  for (int i = 1; i < u.cols; ++i) m = fmaxf(m, scratch[i]);
  __syncthreads();
  scratch[col] = expf(scratch[col] - m);
  __syncthreads();
  float s = 0.0f;
  for (int j = 0; j < u.cols; ++j) s = s + scratch[j];
  __syncthreads();
  out[start + col] = scratch[col] / s;
}}
"""


def test_hiprtc_user_kernels_v1_and_v2(rt):
    ids = (C.c_uint64 * 3)(7001, 7002, 7003)
    srcs = (C.c_char_p * 3)(SIGMOID_BACKWARD_HIP.format(id=7001).encode(), SOFTMAX_V2_HIP.format(id=7002).encode(),
                            SIGMOID_BACKWARD_HIP.format(id=7003).encode())  # same body: served from the cache
    rt.L.malus_runtime_init(ids, srcs, 3)
    assert not rt.L.malus_kernel_is_builtin(7001)
    g, s = RNG.standard_normal(777).astype(np.float32), RNG.uniform(0, 1, 777).astype(np.float32)
    hg, hs = rt.tensor(g), rt.tensor(s)
    for kid_ in (7001, 7003):
        h = rt.L.kernel_dispatch(kid_, M.handles([hg, hs]), 2)
        assert_bitexact(rt.numpy(h), (g * s) * (np.float32(1) - s), "sigmoid_backward")
        rt.free(h)
    x = np.array([[1, 2, 3, 4, 5, 6, 7, 8], [8, 7, 6, 5, 4, 3, 2, 1], [1] * 8,
                  [.1, .9, .2, .8, .3, .7, .4, .6]], np.float32)
    hx = rt.tensor(x)
    ho = rt.L.kernel_dispatch_v2(7002, M.handles([hx]), 1, M.sizes([4, 1, 1]), M.sizes([8, 1, 1]), M.sizes([4, 8]), 2,
                                 0, struct.pack("<i", 8), 4)
    assert_normwise(rt.numpy(ho), O.softmax(x, 1), 1e-5, "user softmax")
    rt.free(hg, hs, hx, ho)


def test_foreign_backward_slot_error_comes_back_as_a_value(rt):
    """A registered backward function may be foreign code (the JIT's own
    VJPs, here a ctypes callback): no exception may cross it.  An entry point
    it calls that fails returns a null handle to it, and backward reports the
    slot's failure with the inner message (return-error mode)."""
    L = rt.L
    RELU_BWD = 9  # BwdSlot numbering, tape.rs:92-175
    FN2 = C.CFUNCTYPE(C.c_int64, C.c_int64, C.c_int64)
    a, b = rt.tensor(np.ones((2, 3), np.float32)), rt.tensor(np.ones((4, 5), np.float32))
    seen = []

    def foreign(dout, x):
        seen.append((dout, x))
        return L.tensor_matmul(a, b)  # fails: inner dims 3 != 4

    cb = FN2(foreign)
    prev = L.malus_tape_backward_fn(RELU_BWD)
    L.tape_reset()
    x = rt.tensor(np.array([-1.0, 2.0, 3.0], np.float32))
    L.tape_register_leaf(x)
    r = L.malus_std_unary(M.RELU, x)
    L.tape_record_unary(OP["Relu"], x, r)
    L.tape_register_backward_fn(RELU_BWD, C.cast(cb, C.c_void_p).value)
    L.malus_set_abort_on_error(0)
    try:
        L.backward(r)
        err = rt.last_error()
        L.malus_clear_error()
    finally:
        L.malus_set_abort_on_error(1)
        L.tape_register_backward_fn(RELU_BWD, prev)
        L.tape_reset()
    assert len(seen) == 1
    assert "backward slot 9 failed" in err and "matmul shape mismatch" in err, err
    # the library is usable afterwards, and the default slot is back
    y = L.malus_std_unary(M.RELU, x)
    assert np.array_equal(rt.numpy(y), [0.0, 2.0, 3.0])
    rt.free(a, b, x, r, y)
