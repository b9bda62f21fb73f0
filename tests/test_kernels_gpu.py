"""GPU parity tests: each stdlib op through the C ABI vs the CPU oracle.

Run on the MI355X box (``-m gpu``).  Inputs are seeded; sizes keep the oracle
in seconds.  Tolerances: see tests/helpers.py.
"""
import ctypes as C
import itertools

import numpy as np
import pytest

import malus_amd as M
from oracle import oracle as O
from tests.helpers import KATS, assert_bitexact, assert_normwise, assert_reduction, assert_ulp

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(1234)


def rand(*shape, lo=-1.0, hi=1.0):
    return RNG.uniform(lo, hi, size=shape).astype(np.float32)


def run(rt, h):
    out = rt.numpy(h)
    rt.free(h)
    return out


# ---------------------------------------------------------------- elementwise
@pytest.mark.parametrize("op", [M.ADD, M.SUB, M.MUL, M.DIV])
@pytest.mark.parametrize("shapes", [((1000003,), (1000003,)), ((257, 64), (64,)), ((6, 5, 7), (5, 7)),
                                    ((384, 16, 16), (16, 16)), ((33, 65), (1, 65)), ((8, 9, 10), (1, 1)),
                                    ((4, 1, 3), (5, 1)), ((1, 4), (3, 4)), ((7,), (3, 7))])
def test_broadcast_binop(rt, op, shapes):
    a, b = rand(*shapes[0]), rand(*shapes[1], lo=0.5, hi=2.0)
    ha, hb = rt.tensor(a), rt.tensor(b)
    got = run(rt, rt.L.malus_std_broadcast_fwd(op, ha, hb))
    want = O.broadcast(op, a, b)
    assert_bitexact(got, want, f"op {op} {shapes}")
    rt.free(ha, hb)


@pytest.mark.parametrize("big,small", [((64, 384), (384,)), ((64, 384), (1, 384)), ((6, 40, 52), (1, 1)),
                                       ((3, 5, 7), (5, 1)), ((4, 8, 16), (1, 8, 1)), ((1, 5), (5,)), ((33, 70001), (1, 1)),
                                       ((5000, 8192), (1, 8192))])
def test_mul_vjp_fused_reduction_matches_materialized(rt, big, small):
    """The broadcast-multiply VJP reduces dout * a without materializing the
    product; it must equal broadcast_mul then sum_to_shape bit for bit, and
    the oracle's sum_to_shape of the product to the reduction bar."""
    dout, a, b = rand(*big), rand(*big), rand(*small)
    hd, ha, hb = rt.tensor(dout), rt.tensor(a), rt.tensor(b)
    fused_b = run(rt, rt.L.malus_std_mul_bwd_b(hd, ha, hb))
    fused_a = run(rt, rt.L.malus_std_mul_bwd_a(hd, hb, ha))  # roles swapped: grad of the broadcast operand
    full = rt.L.malus_std_broadcast_fwd(M.MUL, hd, ha)
    ref = run(rt, rt.L.malus_std_sum_to_shape_bwd(full, hb))
    assert_bitexact(fused_b, ref, f"mul_bwd_b {big} {small}")
    assert_bitexact(fused_a, ref, f"mul_bwd_a {big} {small}")
    prod = dout * a  # f32 products, as the kernel rounds them
    want = O.sum_to_shape(prod, small)
    pad = (1,) * (len(big) - len(small)) + tuple(small)
    axes = tuple(i for i in range(len(big)) if pad[i] == 1 and big[i] != 1)
    exact = prod.astype(np.float64).sum(axis=axes, keepdims=True).reshape(small)
    assert_reduction(fused_b, want, exact, 1e-5, f"vs oracle {big} {small}")
    rt.free(hd, ha, hb, full)


def test_broadcast_operand_swap_quirk(rt):
    # broadcast_binop.ml:90-112: rank(a) < rank(b) computes b - a
    a, b = rand(8), rand(4, 8)
    ha, hb = rt.tensor(a), rt.tensor(b)
    got = run(rt, rt.L.malus_std_broadcast_fwd(M.SUB, ha, hb))
    assert_bitexact(got, b - a, "swapped sub")
    rt.free(ha, hb)


@pytest.mark.parametrize("op,right", [(M.ADD, 1), (M.SUB, 1), (M.SUB, 0), (M.MUL, 1), (M.DIV, 1), (M.DIV, 0)])
def test_scalar_ops(rt, op, right):
    a = rand(100001, lo=0.25, hi=4.0)
    ha = rt.tensor(a)
    got = run(rt, rt.L.malus_std_scalar_op(op, ha, C.c_float(0.37), right))
    assert_bitexact(got, O.scalar_op(op, a, np.float32(0.37), bool(right)), f"scalar op {op} right={right}")
    rt.free(ha)


@pytest.mark.parametrize("op,lo,hi,ulp", [(M.RELU, -3, 3, 0), (M.ABS, -3, 3, 0), (M.SQRT, 0, 100, 0),
                                          (M.EXP, -20, 20, 2), (M.LOG, 1e-3, 1e3, 2), (M.TANH, -6, 6, 2),
                                          (M.SIGMOID, -20, 20, 2)])
def test_unary(rt, op, lo, hi, ulp):
    x = rand(262147, lo=lo, hi=hi)
    hx = rt.tensor(x)
    got = run(rt, rt.L.malus_std_unary(op, hx))
    assert_ulp(got, O.unary(op, x), ulp, f"unary {op}")
    rt.free(hx)


def test_gelu_fwd_bwd(rt):
    # GELU = 0.5x(1 + tanh(g)): a 1-ulp difference in tanh near t = -1 is
    # amplified by the cancellation in (1 + t); the bound is 2 ulp of the
    # result plus the propagated 2-ulp tanh uncertainty 0.5|x| * 2ulp(1).
    x = rand(200003, lo=-8, hi=8)
    hx = rt.tensor(x)
    got = run(rt, rt.L.malus_std_gelu_fwd(hx))
    want = O.unary(O.GELU, x)
    bound = 2 * np.spacing(np.abs(want)) + 0.5 * np.abs(x) * 2 * np.spacing(np.float32(1.0)) * 2
    assert np.all(np.abs(got - want) <= bound), "gelu beyond the derived bound"
    d = rand(200003)
    hd = rt.tensor(d)
    gb = run(rt, rt.L.malus_std_gelu_bwd(hx, hd))
    wb = O.unary_bwd(O.GELU, x, d)
    assert_normwise(gb, wb, 1e-5, "gelu bwd")
    rt.free(hx, hd)


@pytest.mark.parametrize("fn,op", [("malus_std_sigmoid_bwd", O.SIGMOID), ("malus_std_relu_bwd", O.RELU),
                                   ("malus_std_tanh_bwd", O.TANH), ("malus_std_sqrt_bwd", O.SQRT),
                                   ("malus_std_abs_bwd", O.ABS)])
def test_unary_vjp_bitexact(rt, fn, op):
    v = rand(65539, lo=0.1 if op == O.SQRT else -2, hi=2)
    d = rand(65539)
    hv, hd = rt.tensor(v), rt.tensor(d)
    got = run(rt, getattr(rt.L, fn)(hv, hd))
    assert_bitexact(got, O.unary_bwd(op, v, d), fn)
    rt.free(hv, hd)


# ---------------------------------------------------------------- reductions
@pytest.mark.parametrize("shape,axis", [((65, 1024), 1), ((65, 1024), 0), ((3, 70001), 1), ((70001, 3), 0),
                                        ((4, 5, 6), 1), ((4, 5, 6), 2), ((4, 5, 6), 0), ((2, 300, 50), -2), ((4096, 384), 0),
                                        ((3, 999, 40), 1),
                                        # wide rows: the column reduction's contiguous row runs (split into
                                        # chunks with a short last one, and unsplit over many columns)
                                        ((5000, 8192), 0), ((2, 9000, 4096), 1), ((40, 160, 8192), 1),
                                        ((1, 1), 0), ((17,), 0)])
@pytest.mark.parametrize("op", [M.R_SUM, M.R_MEAN, M.R_MAX, M.R_VAR])
def test_reduce_axis(rt, shape, axis, op):
    x = rand(*shape, lo=-2, hi=2)
    hx = rt.tensor(x)
    got = run(rt, rt.L.malus_std_reduce_fwd(op, hx, axis, 1))
    want = O.reduce_axis(op, x, axis, keepdim=True)
    if len(shape) == 1:
        want = want.reshape(1)
    if op == M.R_MAX:
        assert_bitexact(got, want, f"max {shape} {axis}")
    else:
        x64 = x.astype(np.float64)
        exact = {M.R_SUM: x64.sum, M.R_MEAN: x64.mean, M.R_VAR: x64.var}[op](axis=axis, keepdims=True)
        assert_reduction(got, want, exact.reshape(want.shape), 1e-5, f"reduce {op} {shape} {axis}")
    rt.free(hx)


@pytest.mark.parametrize("shape,axis,keep", [((5, 24), 1, 1), ((6, 40, 5), 1, 0), ((3000, 7), 0, 1), ((4, 1500), 1, 0),
                                            ((2, 3, 4), 2, 1), ((17,), 0, 0), ((64, 2048), 0, 0)])
@pytest.mark.parametrize("op", [M.R_SUM, M.R_MEAN, M.R_MAX, M.R_VAR])
def test_reduce_axis_vjps(rt, shape, axis, keep, op):
    """malus_std_reduce_{sum,mean,max,var}_axis_bwd (reduce_bwd.ml:40-71) vs
    the oracle: sum, mean and max are single roundings per element
    (bit-exact; max with ties, every tied maximum gets dout); var goes
    through the device mean, so it meets the reduction bar."""
    x = rand(*shape, lo=-2, hi=2)
    if op == M.R_MAX:
        # every reduced line holds its maximum at least twice (first and last position)
        xv = np.moveaxis(x, axis, -1)
        m = xv.max(axis=-1)
        xv[..., 0] = m
        xv[..., -1] = m
        x = np.ascontiguousarray(np.moveaxis(xv, -1, axis))
    hx = rt.tensor(x)
    hy = rt.L.malus_std_reduce_fwd(op, hx, axis, keep)
    y = rt.numpy(hy)
    dout = rand(*y.shape) if y.ndim else rand(1)
    hd = rt.tensor(dout)
    fn = {M.R_SUM: lambda: rt.L.malus_std_reduce_sum_axis_bwd(hx, hd, axis),
          M.R_MEAN: lambda: rt.L.malus_std_reduce_mean_axis_bwd(hx, hd, axis),
          M.R_MAX: lambda: rt.L.malus_std_reduce_max_axis_bwd(hx, hy, hd, axis),
          M.R_VAR: lambda: rt.L.malus_std_reduce_var_axis_bwd(hx, hd, axis)}[op]
    h = fn()
    assert rt.shape(h) == shape
    got = run(rt, h)
    want = O.reduce_axis_bwd(op, x, dout, axis, y if op == M.R_MAX else None)
    if op == M.R_VAR:
        assert_normwise(got, want, 1e-5, f"var VJP {shape} {axis}")
    else:
        assert_bitexact(got, want, f"reduce VJP {op} {shape} {axis}")
    if op == M.R_MAX:
        assert np.count_nonzero(got) > got.size // shape[axis], "the tie case must be exercised"
    rt.free(hx, hy, hd)


def test_reduce_keepdim_shapes(rt):
    x = rand(2, 3)
    hx = rt.tensor(x)
    for axis, keep, shape in [(0, 0, (3,)), (1, 1, (2, 1)), (0, 1, (1, 3)), (-1, 0, (2,))]:
        h = rt.L.malus_std_reduce_fwd(M.R_SUM, hx, axis, keep)
        assert rt.shape(h) == shape
        rt.free(h)
    rt.free(hx)


def test_sum_all_over_1024_cap(rt):
    x = rand(1 << 20)
    hx = rt.tensor(x)
    got = run(rt, rt.L.malus_std_reduce_all_sum_fwd(hx))
    assert_reduction(got, [O.sum_all(x)], [x.astype(np.float64).sum()], 1e-5, "sum_all")
    rt.free(hx)


# ------------------------------------------------------- softmax / layernorm
@pytest.mark.parametrize("shape,axis", [((37, 1024), 1), ((96, 256), 1), ((64, 65), 1), ((3, 5000), 1),
                                        ((5, 7, 9), 1), ((6, 16, 16), 2), ((8, 3), 0)])
def test_softmax_fwd_bwd(rt, shape, axis):
    x = rand(*shape, lo=-4, hi=4)
    d = rand(*shape)
    hx, hd = rt.tensor(x), rt.tensor(d)
    hy = rt.L.malus_std_softmax_fwd(hx, axis)
    y = rt.numpy(hy)
    ys = O.softmax(x, axis)
    assert_normwise(y, ys, 1e-5, "softmax")
    got = run(rt, rt.L.malus_std_softmax_bwd(hy, hd, axis))
    assert_normwise(got, O.softmax_bwd(y, d, axis), 1e-5, "softmax bwd")
    rt.free(hx, hd, hy)


@pytest.mark.parametrize("t,hs,causal", [(256, 64, 1), (256, 64, 0), (128, 64, 1), (64, 32, 1), (64, 32, 0),
                                          (64, 64, 0)])
def test_attn_scores_softmax_equals_composed_ops(rt, t, hs, causal):
    # nanogpt_modular.ml:57-61: softmax((Q @ permute(K, 0, 2, 1)) * scale + mask, axis=2).
    # The fused kernel reproduces the composed ops bit for bit; the causal
    # form skips the key tiles above the diagonal, whose probabilities are +0.
    bh = 7
    q, kk = rand(bh, t, hs, lo=-2, hi=2), rand(bh, t, hs, lo=-2, hi=2)
    mask = O.causal_mask(t) if causal else rand(t, t, lo=-3, hi=3)
    sc = np.array([[1.0 / np.sqrt(hs)]], np.float32)
    hq, hk, hsc, hm = rt.tensor(q), rt.tensor(kk), rt.tensor(sc), rt.tensor(mask)
    fused = run(rt, rt.L.malus_std_attn_scores_softmax(hq, hk, hsc, hm, causal))
    hkt = rt.L.tensor_permute(hk, M.sizes([0, 2, 1]), 3)
    hS = rt.L.tensor_matmul(hq, hkt)
    hSs = rt.L.malus_std_broadcast_fwd(M.MUL, hS, hsc)
    hSm = rt.L.malus_std_broadcast_fwd(M.ADD, hSs, hm)
    composed = run(rt, rt.L.malus_std_softmax_fwd(hSm, 2))
    assert_bitexact(fused, composed, f"fused scores t={t} hs={hs} causal={causal}")
    S = O.matmul(q, O.permute(kk, (0, 2, 1)))
    want = O.softmax(O.broadcast(M.ADD, O.broadcast(M.MUL, S, sc), mask), 2)
    assert_normwise(fused, want, 1e-5, "fused scores vs oracle")
    if causal:
        assert np.all(fused[:, np.triu_indices(t, 1)[0], np.triu_indices(t, 1)[1]] == 0)
    rt.free(hq, hk, hsc, hm, hkt, hS, hSs, hSm)


@pytest.mark.parametrize("t,hs,causal", [(256, 64, 1), (256, 64, 0), (128, 64, 1), (64, 32, 1), (64, 64, 0)])
def test_attn_scores_bwd_equals_composed_ops(rt, t, hs, causal):
    # softmax VJP (transformer_bwd.ml:15-20) of dP = dout @ permute(V, 0, 2, 1),
    # then the scale multiply's VJP (dout * scale): the fused kernel gives the
    # composed ops' values (the causal form stores +0 above the diagonal,
    # where the composed product P * (dP - sum) is +-0)
    bh = 5
    q, kk, v = (rand(bh, t, hs, lo=-2, hi=2) for _ in range(3))
    d = rand(bh, t, hs)
    mask = O.causal_mask(t) if causal else rand(t, t, lo=-3, hi=3)
    sc = np.array([[1.0 / np.sqrt(hs)]], np.float32)
    hq, hk, hv, hd, hsc, hm = (rt.tensor(a) for a in (q, kk, v, d, sc, mask))
    hp = rt.L.malus_std_attn_scores_softmax(hq, hk, hsc, hm, causal)
    fused = run(rt, rt.L.malus_std_attn_scores_bwd(hd, hv, hp, hsc, causal))
    hvt = rt.L.tensor_permute(hv, M.sizes([0, 2, 1]), 3)
    hdp = rt.L.tensor_matmul(hd, hvt)
    hdx = rt.L.malus_std_softmax_bwd(hp, hdp, 2)
    composed = run(rt, rt.L.malus_std_broadcast_fwd(M.MUL, hdx, hsc))
    assert np.array_equal(fused, composed), f"fused scores bwd t={t} hs={hs} causal={causal}"
    if not causal:
        assert_bitexact(fused, composed, "fused scores bwd")
    p = rt.numpy(hp)
    dp = O.matmul(d, O.permute(v, (0, 2, 1)))
    want = O.broadcast(M.MUL, O.softmax_bwd(p, dp, 2), sc)
    assert_normwise(fused, want, 1e-5, "fused scores bwd vs oracle")
    rt.free(hq, hk, hv, hd, hsc, hm, hp, hvt, hdp, hdx)


@pytest.mark.parametrize("t,hs,causal", [(256, 64, 1), (256, 64, 0), (128, 64, 1), (64, 32, 1), (64, 32, 0),
                                          (64, 64, 0)])
def test_attn_fwd_equals_composed_ops(rt, t, hs, causal):
    # nanogpt_modular.ml:57-62: attn @ V with attn the fused scores softmax.
    # P @ V runs from the scores kernel's registers; it equals the batched
    # matmul of the stored P with V bit for bit (a causal P's zeros above the
    # diagonal add exact zeros in the matmul)
    bh = 6
    q, kk, v = (rand(bh, t, hs, lo=-2, hi=2) for _ in range(3))
    mask = O.causal_mask(t) if causal else rand(t, t, lo=-3, hi=3)
    sc = np.array([[1.0 / np.sqrt(hs)]], np.float32)
    hq, hk, hv, hsc, hm = (rt.tensor(a) for a in (q, kk, v, sc, mask))
    hp = C.c_int64()
    fused = run(rt, rt.L.malus_std_attn_fwd(hq, hk, hv, hsc, hm, causal, C.byref(hp)))
    p_fused = run(rt, hp.value)
    hp2 = rt.L.malus_std_attn_scores_softmax(hq, hk, hsc, hm, causal)
    assert_bitexact(p_fused, rt.numpy(hp2), f"attn_fwd P t={t} hs={hs} causal={causal}")
    composed = run(rt, rt.L.tensor_matmul(hp2, hv))
    assert_bitexact(fused, composed, f"attn_fwd P@V t={t} hs={hs} causal={causal}")
    assert_normwise(fused, O.matmul(p_fused, v), 1e-5, "attn_fwd vs oracle matmul")
    rt.free(hq, hk, hv, hsc, hm, hp2)


@pytest.mark.parametrize("t,hs,causal", [(256, 64, 1), (256, 64, 0), (128, 64, 1), (64, 32, 1), (64, 64, 0)])
def test_attn_bwd_dq_equals_composed_ops(rt, t, hs, causal):
    # The scores backward with the Q gradient of the scores product
    # (dQ = dS @ K) run from the same kernel's registers: dS equals the
    # scores backward alone and dQ the batched matmul of that dS with K
    bh = 5
    q, kk, v = (rand(bh, t, hs, lo=-2, hi=2) for _ in range(3))
    d = rand(bh, t, hs)
    mask = O.causal_mask(t) if causal else rand(t, t, lo=-3, hi=3)
    sc = np.array([[1.0 / np.sqrt(hs)]], np.float32)
    hq, hk, hv, hd, hsc, hm = (rt.tensor(a) for a in (q, kk, v, d, sc, mask))
    hp = rt.L.malus_std_attn_scores_softmax(hq, hk, hsc, hm, causal)
    hdq = C.c_int64()
    ds = run(rt, rt.L.malus_std_attn_bwd(hd, hv, hp, hsc, hk, causal, C.byref(hdq)))
    dq = run(rt, hdq.value)
    hds2 = rt.L.malus_std_attn_scores_bwd(hd, hv, hp, hsc, causal)
    assert_bitexact(ds, rt.numpy(hds2), f"attn_bwd dS t={t} hs={hs} causal={causal}")
    composed = run(rt, rt.L.tensor_matmul(hds2, hk))
    assert_bitexact(dq, composed, f"attn_bwd dQ t={t} hs={hs} causal={causal}")
    assert_normwise(dq, O.matmul(ds, kk), 1e-5, "attn_bwd dQ vs oracle matmul")
    rt.free(hq, hk, hv, hd, hsc, hm, hp, hds2)


@pytest.mark.parametrize("t,hs,causal,bh", [(256, 64, 1, 5), (256, 64, 0, 5), (128, 64, 1, 5), (64, 32, 1, 5),
                                             (64, 64, 0, 5), (256, 64, 1, 300), (64, 32, 0, 600)])
def test_attn_bwd_all_equals_composed_ops(rt, t, hs, causal, bh):
    # The whole attention VJP from one kernel: dS and dQ as the kernel
    # without the key-side products; dK and dV as the composed ops of
    # nanogpt_modular.ml:54-61 form them: dK = (Q^T @ dS)^T (the VJP of
    # Q @ Kt with respect to Kt, permuted back) and dV = P^T @ dO (the VJP
    # of attn @ V with respect to V), every output bit-exact.
    # Up to 600 heads: more workgroups than CUs.
    q, kk, v = (rand(bh, t, hs, lo=-2, hi=2) for _ in range(3))
    d = rand(bh, t, hs)
    mask = O.causal_mask(t) if causal else rand(t, t, lo=-3, hi=3)
    sc = np.array([[1.0 / np.sqrt(hs)]], np.float32)
    hq, hk, hv, hd, hsc, hm = (rt.tensor(a) for a in (q, kk, v, d, sc, mask))
    hp = rt.L.malus_std_attn_scores_softmax(hq, hk, hsc, hm, causal)
    hdq, hdk, hdv = C.c_int64(), C.c_int64(), C.c_int64()
    ds = run(rt, rt.L.malus_std_attn_bwd_all(hd, hq, hk, hv, hp, hsc, causal, 0, 0, 0, C.byref(hdq), C.byref(hdk),
                                             C.byref(hdv)))
    dq, dk, dv = (run(rt, h.value) for h in (hdq, hdk, hdv))
    # with addends (an existing gradient of each input): each output is the
    # f32 sum of the addend and the product
    adds = [rand(bh, t, hs) for _ in range(3)]
    ha = [rt.tensor(a) for a in adds]
    run(rt, rt.L.malus_std_attn_bwd_all(hd, hq, hk, hv, hp, hsc, causal, ha[0], ha[1], ha[2], C.byref(hdq),
                                        C.byref(hdk), C.byref(hdv)))
    for name, h, a, base in zip("QKV", (hdq, hdk, hdv), adds, (dq, dk, dv)):
        assert_bitexact(run(rt, h.value), a + base, f"attn_bwd_all d{name} with addend")
    rt.free(*ha)
    hdq2 = C.c_int64()
    hds2 = rt.L.malus_std_attn_bwd(hd, hv, hp, hsc, hk, causal, C.byref(hdq2))
    tag = f"t={t} hs={hs} causal={causal}"
    assert_bitexact(ds, rt.numpy(hds2), f"attn_bwd_all dS {tag}")
    assert_bitexact(dq, run(rt, hdq2.value), f"attn_bwd_all dQ {tag}")
    hqt = rt.L.tensor_permute(hq, M.sizes([0, 2, 1]), 3)
    hpt = rt.L.tensor_permute(hp, M.sizes([0, 2, 1]), 3)
    hdkt = rt.L.tensor_matmul(hqt, hds2)
    assert_bitexact(dk, run(rt, rt.L.tensor_permute(hdkt, M.sizes([0, 2, 1]), 3)), f"attn_bwd_all dK {tag}")
    assert_bitexact(dv, run(rt, rt.L.tensor_matmul(hpt, hd)), f"attn_bwd_all dV {tag}")
    p = rt.numpy(hp)
    assert_normwise(dk, O.matmul(np.ascontiguousarray(ds.transpose(0, 2, 1)), q), 1e-5, "dK vs oracle matmul")
    assert_normwise(dv, O.matmul(np.ascontiguousarray(p.transpose(0, 2, 1)), d), 1e-5, "dV vs oracle matmul")
    rt.free(hq, hk, hv, hd, hsc, hm, hp, hds2, hqt, hdkt, hpt)


def test_attn_scores_softmax_rejects_unbuilt_shapes(rt):
    hq = rt.tensor(rand(2, 48, 16))
    hsc, hm = rt.tensor(np.ones((1, 1), np.float32)), rt.tensor(O.causal_mask(48))
    rt.L.malus_set_abort_on_error(0)
    try:
        assert rt.L.malus_std_attn_scores_softmax(hq, hq, hsc, hm, 1) == 0
        assert "no fused kernel" in rt.last_error()
        rt.L.malus_clear_error()
        assert rt.L.malus_std_attn_fwd(hq, hq, hq, hsc, hm, 1, None) == 0
        assert "no fused kernel" in rt.last_error()
        rt.L.malus_clear_error()
        hp = rt.tensor(rand(2, 48, 48))
        assert rt.L.malus_std_attn_bwd(hq, hq, hp, hsc, hq, 1, None) == 0
        assert "no fused kernel" in rt.last_error()
        rt.L.malus_clear_error()
        hv = rt.tensor(rand(2, 48, 32))  # v of another head size
        assert rt.L.malus_std_attn_fwd(hq, hq, hv, hsc, hm, 1, None) == 0
        assert "attn_fwd shape mismatch" in rt.last_error()
        rt.L.malus_clear_error()
        rt.free(hp, hv)
    finally:
        rt.L.malus_set_abort_on_error(1)
    rt.free(hq, hsc, hm)


def test_attn_causal_flag_requires_causal_operands(rt):
    # causal=1 skips the key tiles above the diagonal: valid only for the
    # causal mask itself and, in the VJPs, for P written by a causal forward.
    # Anything else is an error, never a silently wrong result.
    t, hs = 64, 32
    hq = rt.tensor(rand(3, t, hs))
    hsc = rt.tensor(np.ones((1, 1), np.float32))
    hm_bad = rt.tensor(rand(t, t))
    hm_ok = rt.L.tensor_causal_mask(t)
    hi = rt.tensor(np.zeros((3, t, hs), np.int32))
    rt.L.malus_set_abort_on_error(0)
    try:
        assert rt.L.malus_std_attn_scores_softmax(hq, hq, hsc, hm_bad, 1) == 0
        assert "causal=1 needs the causal mask" in rt.last_error()
        rt.L.malus_clear_error()
        assert rt.L.malus_std_attn_fwd(hq, hq, hq, hsc, hm_bad, 1, None) == 0
        assert "causal=1 needs the causal mask" in rt.last_error()
        rt.L.malus_clear_error()
        hp_dense = rt.L.malus_std_attn_scores_softmax(hq, hq, hsc, hm_bad, 0)
        assert hp_dense != 0
        assert rt.L.malus_std_attn_bwd(hq, hq, hp_dense, hsc, hq, 1, None) == 0
        assert "written by a causal attention forward" in rt.last_error()
        rt.L.malus_clear_error()
        assert rt.L.malus_std_attn_scores_bwd(hq, hq, hp_dense, hsc, 1) == 0
        assert "written by a causal attention forward" in rt.last_error()
        rt.L.malus_clear_error()
        assert rt.L.malus_std_attn_fwd(hi, hq, hq, hsc, hm_ok, 1, None) == 0
        assert "must be f32" in rt.last_error()
        rt.L.malus_clear_error()
        hp_causal = rt.L.malus_std_attn_scores_softmax(hq, hq, hsc, hm_ok, 1)
        hds = rt.L.malus_std_attn_scores_bwd(hq, hq, hp_causal, hsc, 1)
        assert hds != 0, rt.last_error()
        rt.free(hp_dense, hp_causal, hds)
    finally:
        rt.L.malus_set_abort_on_error(1)
    rt.free(hq, hsc, hm_bad, hm_ok, hi)


@pytest.mark.parametrize("shape,axis", [((65, 1024), 1), ((100, 384), 1), ((33, 128), 1), ((4, 70), 1),
                                        ((3, 5000), 1), ((6, 8, 5), 1)])
def test_layernorm_fwd_bwd(rt, shape, axis):
    x = rand(*shape, lo=-3, hi=3) + 0.5
    d = rand(*shape)
    hx, hd = rt.tensor(x), rt.tensor(d)
    hv = C.c_int64()
    hy = rt.L.malus_std_layernorm_fwd(hx, axis, C.byref(hv))
    y, var = rt.numpy(hy), rt.numpy(hv.value)
    ys, vs = O.layernorm(x, axis)
    assert_normwise(y, ys, 1e-5, "layernorm y")
    assert_normwise(var, vs, 1e-5, "layernorm var")
    assert var.shape == vs.shape
    got = run(rt, rt.L.malus_std_layernorm_bwd(hy, hv.value, hd, axis))
    assert_normwise(got, O.layernorm_bwd(y, var, d, axis), 1e-5, "layernorm bwd")
    rt.free(hx, hd, hy, hv.value)


def test_layernorm_kat(rt):
    # metal_integration.rs:296-301 inputs
    x = np.array([[1, 2, 3, 4, 5, 6, 7, 8], [.1, .2, .3, .4, .5, .6, .7, .8],
                  [-3, -2, -1, 0, 1, 2, 3, 4], [10, 10.1, 9.9, 10.2, 9.8, 10.3, 9.7, 10.4]], np.float32)
    hx = rt.tensor(x)
    hy = rt.L.malus_std_layernorm_fwd(hx, 1, None)
    got = run(rt, hy)
    mu = x.mean(1, keepdims=True, dtype=np.float64)
    ref = (x - mu) / np.sqrt(x.var(1, keepdims=True, dtype=np.float64) + 1e-5)
    assert np.max(np.abs(got - ref)) < 1e-5
    rt.free(hx)


@pytest.mark.parametrize("n,v", [(50, 65), (20, 1024), (7, 5000)])
def test_cross_entropy_fwd_bwd(rt, n, v):
    logits = (RNG.standard_normal((n, v)) * 2).astype(np.float32)
    t = RNG.integers(0, v, n).astype(np.int32)
    hl, ht = rt.tensor(logits), rt.tensor(t)
    hp = C.c_int64()
    hloss = rt.L.malus_std_cross_entropy_fwd(hl, ht, C.byref(hp))
    loss, probs = rt.numpy(hloss), rt.numpy(hp.value)
    wl, wp = O.cross_entropy(logits, t)
    assert_normwise(probs, wp, 1e-5, "probs")
    assert_normwise(loss, np.array([wl]), 1e-5, "loss")
    hd = rt.tensor(np.array([1.0], np.float32))
    got = run(rt, rt.L.malus_std_cross_entropy_bwd(hp.value, ht, hd))
    assert_normwise(got, O.cross_entropy_bwd(probs, t, 1.0), 1e-6, "ce bwd")
    rt.free(hl, ht, hloss, hp.value, hd)


# ------------------------------------------------------------ index ops
@pytest.mark.parametrize("v,d,t", [(65, 384, 4096), (256, 384, 2048), (65, 65, 777), (4, 3, 4), (3, 128, 16384),
                                   (65, 384, 4097), (2048, 64, 9000), (400, 32, 4096), (65, 384, 16384), (256, 384, 16384),
                                   (1000, 36, 500), (5, 100, 40001)])
def test_embedding_fwd_bwd_bitexact(rt, v, d, t):
    w = rand(v, d)
    idx = RNG.integers(0, v, t).astype(np.int32)
    dout = rand(t, d)
    hw, hi, hd = rt.tensor(w), rt.tensor(idx), rt.tensor(dout)
    got = run(rt, rt.L.malus_std_embedding_fwd(hw, hi))
    assert_bitexact(got, O.embedding(w, idx), "embedding")
    gb = run(rt, rt.L.malus_std_embedding_bwd(hw, hi, hd))
    assert_bitexact(gb, O.embedding_bwd(dout, idx, v), "embedding bwd (token-ordered sums)")
    rt.free(hw, hi, hd)


@pytest.mark.parametrize("counts,v", [
    ([256, 257, 0, 255, 512, 1, 2000], 7),      # mean t / v = 468: 256-token chunks
    ([64, 65, 128, 129, 0, 1, 63, 200], 16),    # mean 40 (rows 8..15 unused): 64-token chunks
    ([96, 97, 33, 0, 160], 5),                  # mean 77: 128-token chunks
], ids=["chunk256", "chunk64", "chunk128"])
def test_embedding_bwd_chunk_boundaries(rt, counts, v):
    # The VJP stages each vocabulary row's listed tokens through LDS in
    # chunks of 64, 128 or 256 (chosen from the mean list length t / v):
    # rows whose lists end on, just past and just short of a chunk, empty
    # rows, and one long row, with the tokens of all rows interleaved, must
    # give the token-ordered sums bit for bit.
    rng = np.random.default_rng(len(counts))
    idx = np.concatenate([np.full(c, r, np.int32) for r, c in enumerate(counts)])
    rng.shuffle(idx)
    t, d = len(idx), 100  # d: three 32-column blocks and a 4-column tail
    w = rand(v, d)
    dout = rand(t, d)
    hw, hi, hd = rt.tensor(w), rt.tensor(idx), rt.tensor(dout)
    gb = run(rt, rt.L.malus_std_embedding_bwd(hw, hi, hd))
    assert_bitexact(gb, O.embedding_bwd(dout, idx, v), f"embedding bwd, row counts {counts}")
    rt.free(hw, hi, hd)


def test_embedding_kat(rt):
    for kat in KATS["embedding"]:
        hw, hi = rt.tensor(np.array(kat["w"], np.float32)), rt.tensor(np.array(kat["idx"], np.int32))
        assert_bitexact(run(rt, rt.L.malus_std_embedding_fwd(hw, hi)), np.array(kat["out"], np.float32), kat["source"])
        rt.free(hw, hi)
    kat = KATS["embedding_bwd_counts"]
    hw = rt.tensor(np.zeros((kat["vocab"], 3), np.float32))
    hd = rt.tensor(np.ones((len(kat["idx"]), 3), np.float32))
    hi = rt.tensor(np.array(kat["idx"], np.int32))
    g = run(rt, rt.L.malus_std_embedding_bwd(hw, hi, hd))
    assert g[:, 0].tolist() == kat["row_counts"] and np.all(g == g[:, :1])
    rt.free(hw, hd, hi)


@pytest.mark.parametrize("perm", list(itertools.permutations(range(4))))
def test_permute_4d_bitexact(rt, perm):
    x = rand(3, 4, 5, 8)
    hx = rt.tensor(x)
    got = run(rt, rt.L.tensor_permute(hx, M.sizes(perm), 4))
    assert_bitexact(got, O.permute(x, perm), f"perm {perm}")
    rt.free(hx)


@pytest.mark.parametrize("shape", [(65, 130), (1, 7), (384, 64), (129, 257)])
def test_transpose_2d(rt, shape):
    x = rand(*shape)
    hx = rt.tensor(x)
    got = run(rt, rt.L.malus_std_transpose_2d_fwd(hx))
    assert_bitexact(got, x.T.copy(), "transpose")
    rt.free(hx)


def test_permute_3d_batched_transpose(rt):
    x = rand(384, 64, 256)
    hx = rt.tensor(x)
    got = run(rt, rt.L.malus_std_permute_3d_fwd(hx, 0, 2, 1))
    assert_bitexact(got, np.ascontiguousarray(x.transpose(0, 2, 1)), "permute(0,2,1)")
    rt.free(hx)


# ------------------------------------------------------------------- matmul
MM_SHAPES = [((2, 3), (3, 2)), ((1, 1), (1, 1)), ((65, 127), (127, 129)), ((128, 128), (128, 128)),
             ((300, 384), (384, 65)), ((4, 8), (8, 1)), ((8, 64, 32), (8, 32, 48)), ((3, 5, 7), (7, 9)),
             ((384, 1024), (1024, 384)), ((16384, 4), (4, 8))]


@pytest.mark.parametrize("sa,sb", MM_SHAPES)
def test_matmul_and_vjps(rt, sa, sb):
    a, b = rand(*sa), rand(*sb)
    ha, hb = rt.tensor(a), rt.tensor(b)
    hc = rt.L.tensor_matmul(ha, hb)
    c = rt.numpy(hc)
    assert_normwise(c, O.matmul(a, b), 1e-5, f"matmul {sa}@{sb}")
    d = rand(*c.shape)
    hd = rt.tensor(d)
    da = run(rt, rt.L.malus_std_matmul_bwd_a(ha, hb, hd))
    db = run(rt, rt.L.malus_std_matmul_bwd_b(ha, hb, hd))
    bt = O.permute(b, (0, 2, 1)) if b.ndim == 3 else O.permute(b, (1, 0))
    wa = O.matmul(d, bt)
    if a.ndim == 3 and b.ndim == 2:
        # matmul_bwd.ml:28-29: reduce_sum(permute(a) @ dC, 0)
        wb = O.reduce_axis(O.R_SUM, O.matmul(O.permute(a, (0, 2, 1)), d), 0)
    elif a.ndim == 3:
        wb = O.matmul(O.permute(a, (0, 2, 1)), d)
    else:
        wb = O.matmul(O.permute(a, (1, 0)), d)
    assert_normwise(da, wa.reshape(a.shape), 1e-5, "dA")
    assert_normwise(db, wb.reshape(b.shape), 1e-5, "dB")
    rt.free(ha, hb, hc, hd)


def test_matmul_kats(rt):
    for kat in KATS["matmul"]:
        ha, hb = rt.tensor(np.array(kat["a"], np.float32)), rt.tensor(np.array(kat["b"], np.float32))
        assert_bitexact(run(rt, rt.L.tensor_matmul(ha, hb)), np.array(kat["out"], np.float32), kat["source"])
        rt.free(ha, hb)
    o1 = rt.L.tensor_alloc_ones_gpu(M.sizes([2, 3]), 2)
    o2 = rt.L.tensor_alloc_ones_gpu(M.sizes([3, 4]), 2)
    out = run(rt, rt.L.tensor_matmul(o1, o2))
    assert out.shape == (2, 4) and np.all(out == 3.0)
    rt.free(o1, o2)
    # kernel -> matmul -> kernel with one flush at the read
    kat = KATS["add_matmul_add_chain"]
    ha = rt.tensor(np.array(kat["a"], np.float32))
    x = rt.L.malus_std_broadcast_fwd(M.ADD, ha, ha)
    y = rt.L.tensor_matmul(x, x)
    z = rt.L.malus_std_broadcast_fwd(M.ADD, y, y)
    assert rt.L.tensor_is_pending(z)
    assert_bitexact(run(rt, z), np.array(kat["out"], np.float32), kat["source"])
    rt.free(ha, x, y)


@pytest.mark.parametrize("kat", KATS["reduce"], ids=lambda k: k["op"] + str(k["axis"]))
def test_reduce_kats(rt, kat):
    op = {"sum": M.R_SUM, "mean": M.R_MEAN, "max": M.R_MAX, "var": M.R_VAR}[kat["op"]]
    hx = rt.tensor(np.array(kat["x"], np.float32))
    got = run(rt, rt.L.malus_std_reduce_fwd(op, hx, kat["axis"], kat["keepdim"]))
    assert_bitexact(got, np.array(kat["out"], np.float32), kat["source"])
    rt.free(hx)


def test_matmul_split_k_weight_grad_shape(rt):
    # dW of a C5 projection: [384, 16384] @ [16384, 384] through the TN path
    x = rand(16384, 384)
    d = rand(16384, 384)
    w = rand(384, 384)
    hx, hd, hw = rt.tensor(x), rt.tensor(d), rt.tensor(w)
    got = run(rt, rt.L.malus_std_matmul_bwd_b(hx, hw, hd))
    O.set_threads(8)
    want = O.matmul(O.permute(x, (1, 0)), d)
    assert_normwise(got, want, 1e-5, "split-K dW")
    rt.free(hx, hd, hw)


@pytest.mark.parametrize("m,n", [(41, 35), (64, 36)])
def test_matmul_split_k_reduce_widths(rt, m, n):
    # long K with few output tiles takes the split-K path; an output whose
    # size is not a multiple of 4 uses the scalar partial reduction, the
    # others the float4 one
    x = rand(8192, m)
    d = rand(8192, n)
    w = rand(m, n)
    hx, hd, hw = rt.tensor(x), rt.tensor(d), rt.tensor(w)
    got = run(rt, rt.L.malus_std_matmul_bwd_b(hx, hw, hd))
    want = O.matmul(O.permute(x, (1, 0)), d)
    assert_normwise(got, want, 1e-5, "split-K dW")
    rt.free(hx, hd, hw)


# ---------------------------------------------------------------- optimizer
def test_adam_l2_fused_bitexact(rt):
    n = 100003
    p, g, m = rand(n), rand(n), rand(n) * 0.1
    v = np.abs(rand(n)) * 0.01
    hs = [rt.tensor(a) for a in (p, g, m, v)]
    mo, vo = C.c_int64(), C.c_int64()
    for t in (1, 7):
        hp = rt.L.malus_std_adam_l2(*hs, 1e-3, 0.9, 0.99, 1e-8, 0.1, t, C.byref(mo), C.byref(vo))
        wp, wm, wv = O.adam_l2(p, g, m, v, 1e-3, 0.9, 0.99, 1e-8, 0.1, t)
        assert_bitexact(run(rt, hp), wp, "p'")
        assert_bitexact(run(rt, mo.value), wm, "m'")
        assert_bitexact(run(rt, vo.value), wv, "v'")
    rt.free(*hs)
