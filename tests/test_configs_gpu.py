"""The C2 and C3 workloads as programs through the tape (their composed
chains, not each op on its own), and C5 over several steps.

C2: z = a*b + 0.5*c - relu(a) and a [R,C] + [1,C] row
broadcast, forward and backward.  The tensor-scalar product `0.5*c` records
no tape node (codegen-cpu/src/lib.rs:1556-1580), so c receives no gradient;
the other gradients are sums of +-1, b and a and come out bit-exact.

Both run at the configuration's own [8192, 8192] and at 1/64 of it.

C3, at [65536, 1024]: layernorm with gamma = 1 and beta = 0
perturbed by N(0, 0.02) (nanogpt_modular.ml:38-45 applies the weight as a
broadcast mul), through the tape with a random upstream gradient: normwise
1e-5 against the oracle's composition of the same VJPs (also at 4,096 rows);
softmax, GELU and cross-entropy (logits ~ N(0, 2), int32 targets in
[0, 1024)) forward and backward, and the axis-0 and axis-1 sums, against the
oracle at the bars of tests/helpers.py.

C5: three training steps (loss within 1e-5 relative each step;
after the third, at most 0.1% of the parameters more than 1e-5 apart)."""
import ctypes as C
import os

import numpy as np
import pytest

import malus_amd as M
from oracle import oracle as O
from tests.helpers import assert_bitexact, assert_normwise, assert_reduction, normwise_err

pytestmark = pytest.mark.gpu

OP = dict(Matmul=0, Add=1, Sub=2, Mul=3, Div=4, Relu=6, Sum=12, Layernorm=21)
C5 = dict(V=65, T=256, C=384, H=6, L=6, B=64)
OPT = dict(lr=1e-3, b1=0.9, b2=0.99, eps=1e-8, wd=0.1)


@pytest.fixture
def tape(rt):
    rt.L.tape_reset()
    yield rt
    rt.L.tape_reset()


def leaf(rt, arr):
    h = rt.tensor(arr)
    rt.L.tape_register_leaf(h)
    return h


def grad(rt, h):
    g = rt.L.tape_get_grad(h)
    if not g:
        return None
    out = rt.numpy(g)
    rt.free(g)
    return out


@pytest.mark.parametrize("R,Cc", [(1024, 1024), (8192, 8192)], ids=["1_64th", "full_2pow26"])
def test_c2_chain_through_the_tape(tape, R, Cc):
    rt = tape
    rng = np.random.default_rng(2)
    a, b, c = (rng.uniform(-1, 1, (R, Cc)).astype(np.float32) for _ in range(3))
    bias = rng.uniform(-1, 1, (1, Cc)).astype(np.float32)
    ha, hb, hc, hbias = leaf(rt, a), leaf(rt, b), leaf(rt, c), leaf(rt, bias)
    ab = rt.L.malus_std_broadcast_fwd(M.MUL, ha, hb)
    rt.L.tape_record_binop(OP["Mul"], ha, hb, ab)
    half_c = rt.L.malus_std_scalar_op(M.MUL, hc, 0.5, 0)  # 0.5*c: no tape node
    s1 = rt.L.malus_std_broadcast_fwd(M.ADD, ab, half_c)
    rt.L.tape_record_binop(OP["Add"], ab, half_c, s1)
    r = rt.L.malus_std_unary(M.RELU, ha)
    rt.L.tape_record_unary(OP["Relu"], ha, r)
    z = rt.L.malus_std_broadcast_fwd(M.SUB, s1, r)
    rt.L.tape_record_binop(OP["Sub"], s1, r, z)
    # the row broadcast of the same config
    y = rt.L.malus_std_broadcast_fwd(M.ADD, z, hbias)
    rt.L.tape_record_binop(OP["Add"], z, hbias, y)

    want_z = O.broadcast(O.SUB, O.broadcast(O.ADD, O.broadcast(O.MUL, a, b), O.scalar_op(O.MUL, c, 0.5, False)),
                         O.unary(O.RELU, a))
    assert_bitexact(rt.numpy(z), want_z, "z")
    assert_bitexact(rt.numpy(y), O.broadcast(O.ADD, want_z, bias), "z + bias")

    rt.L.backward(y)
    # dy = 1: dz = 1; ds1 = 1, dr = -1; da = -(a > 0) + b (Relu, then Mul); db = a; dc: none
    assert_bitexact(grad(rt, ha), (np.float32(-1.0) * (a > 0)).astype(np.float32) + b, "da")
    assert_bitexact(grad(rt, hb), a, "db")
    assert grad(rt, hc) is None or not np.any(grad(rt, hc)), "0.5*c is not taped: c gets no gradient"
    assert_bitexact(grad(rt, hbias), np.full((1, Cc), R, np.float32), "dbias (sum over rows of ones)")
    rt.free(ha, hb, hc, hbias, ab, half_c, s1, r, z, y)


@pytest.mark.parametrize("R", [4096, 65536], ids=["1_16th", "full_65536"])
def test_c3_affine_layernorm_through_the_tape(tape, R):
    rt = tape
    rng = np.random.default_rng(3)
    Cc = 1024
    x = rng.standard_normal((R, Cc)).astype(np.float32)
    gamma = (1.0 + 0.02 * rng.standard_normal(Cc)).astype(np.float32)
    beta = (0.02 * rng.standard_normal(Cc)).astype(np.float32)
    up = rng.uniform(-1, 1, (R, Cc)).astype(np.float32)
    hx, hg, hbeta = leaf(rt, x), leaf(rt, gamma), leaf(rt, beta)
    hup = rt.tensor(up)
    hv = C.c_int64()
    hy = rt.L.malus_std_layernorm_fwd(hx, 1, C.byref(hv))
    rt.L.tape_record_layernorm(OP["Layernorm"], hx, hy, hv.value, 1)  # the tape takes var (tape.rs:289-310)
    hs = rt.L.malus_std_broadcast_fwd(M.MUL, hy, hg)
    rt.L.tape_record_binop(OP["Mul"], hy, hg, hs)
    ho = rt.L.malus_std_broadcast_fwd(M.ADD, hs, hbeta)
    rt.L.tape_record_binop(OP["Add"], hs, hbeta, ho)
    hl = rt.L.malus_std_broadcast_fwd(M.MUL, ho, hup)  # an upstream gradient `up`
    rt.L.tape_record_binop(OP["Mul"], ho, hup, hl)
    rt.L.backward(hl)

    y, var = O.layernorm(x, 1)
    out = O.broadcast(O.ADD, O.broadcast(O.MUL, y, gamma), beta)
    assert_normwise(rt.numpy(ho), out, 1e-5, "gamma * ln(x) + beta")
    # VJPs in the tape's order: Mul(o, up) -> Add -> Mul(y, gamma) -> Layernorm
    d_o = up
    dbeta = O.sum_to_shape(d_o, (Cc,))
    dgamma = O.sum_to_shape(O.broadcast(O.MUL, d_o, y), (Cc,))
    dy = O.broadcast(O.MUL, d_o, gamma)
    dx = O.layernorm_bwd(y, var, dy, 1)
    assert_normwise(grad(rt, hbeta), dbeta, 1e-5, "dbeta")
    assert_normwise(grad(rt, hg), dgamma, 1e-5, "dgamma")
    assert_normwise(grad(rt, hx), dx, 1e-5, "dx")
    rt.free(hx, hg, hbeta, hup, hy, hs, ho, hl)


C3_ROWS, C3_COLS = 65536, 1024


def run(rt, h):
    assert h, rt.last_error()
    out = rt.numpy(h)
    rt.free(h)
    return out


def test_c3_softmax_at_full_size(rt):
    rng = np.random.default_rng(31)
    x = rng.uniform(-4, 4, (C3_ROWS, C3_COLS)).astype(np.float32)
    d = rng.uniform(-1, 1, (C3_ROWS, C3_COLS)).astype(np.float32)
    hx, hd = rt.tensor(x), rt.tensor(d)
    hy = rt.L.malus_std_softmax_fwd(hx, 1)
    y = rt.numpy(hy)
    assert_normwise(y, O.softmax(x, 1), 1e-5, "softmax [65536,1024]")
    assert_normwise(run(rt, rt.L.malus_std_softmax_bwd(hy, hd, 1)), O.softmax_bwd(y, d, 1), 1e-5, "softmax bwd")
    rt.free(hx, hd, hy)


def test_c3_gelu_at_full_size(rt):
    rng = np.random.default_rng(32)
    x = rng.uniform(-8, 8, (C3_ROWS, C3_COLS)).astype(np.float32)
    d = rng.uniform(-1, 1, (C3_ROWS, C3_COLS)).astype(np.float32)
    hx, hd = rt.tensor(x), rt.tensor(d)
    got = run(rt, rt.L.malus_std_gelu_fwd(hx))
    want = O.unary(O.GELU, x)
    # 2 ulp of the result plus the propagated 2-ulp tanh uncertainty 0.5|x| * 2 ulp(1)
    bound = 2 * np.spacing(np.abs(want)) + 0.5 * np.abs(x) * 2 * np.spacing(np.float32(1.0)) * 2
    assert np.all(np.abs(got - want) <= bound), "gelu [65536,1024] beyond the derived bound"
    del got, want, bound
    assert_normwise(run(rt, rt.L.malus_std_gelu_bwd(hx, hd)), O.unary_bwd(O.GELU, x, d), 1e-5, "gelu bwd")
    rt.free(hx, hd)


def test_c3_cross_entropy_at_full_size(rt):
    rng = np.random.default_rng(33)
    logits = (rng.standard_normal((C3_ROWS, C3_COLS)) * 2).astype(np.float32)
    t = rng.integers(0, C3_COLS, C3_ROWS).astype(np.int32)
    hl, ht = rt.tensor(logits), rt.tensor(t)
    hp = C.c_int64()
    hloss = rt.L.malus_std_cross_entropy_fwd(hl, ht, C.byref(hp))
    loss, probs = rt.numpy(hloss), rt.numpy(hp.value)
    wl, wp = O.cross_entropy(logits, t)
    assert_normwise(probs, wp, 1e-5, "probs [65536,1024]")
    # the loss is a mean over 65,536 rows: within 1e-5 of the float64 mean of
    # -log p[target], or no farther from it than the oracle's sequential sum
    exact = -np.mean(np.log(wp[np.arange(C3_ROWS), t].astype(np.float64)))
    assert_reduction(loss, np.array([wl]), np.array([exact]), 1e-5, "ce loss")
    hd = rt.tensor(np.array([1.0], np.float32))
    got = run(rt, rt.L.malus_std_cross_entropy_bwd(hp.value, ht, hd))
    assert_normwise(got, O.cross_entropy_bwd(probs, t, 1.0), 1e-6, "ce bwd")
    rt.free(hl, ht, hloss, hp.value, hd)


@pytest.mark.parametrize("axis", [0, 1])
def test_c3_axis_sums_at_full_size(rt, axis):
    rng = np.random.default_rng(34 + axis)
    x = rng.uniform(-2, 2, (C3_ROWS, C3_COLS)).astype(np.float32)
    hx = rt.tensor(x)
    got = run(rt, rt.L.malus_std_reduce_fwd(M.R_SUM, hx, axis, 0))
    exact = x.astype(np.float64).sum(axis=axis)
    assert_reduction(got, O.reduce_axis(O.R_SUM, x, axis), exact, 1e-5, f"sum over axis {axis} of [65536,1024]")
    rt.free(hx)


def test_c5_three_step_trajectory(rt):
    rt.L.tape_reset()
    rt.L.malus_rng_set_counter(0)
    g = rt.L.malus_gpt_create(C5["V"], C5["T"], C5["C"], C5["H"], C5["L"], C5["B"], OPT["lr"], OPT["b1"],
                              OPT["b2"], OPT["eps"], OPT["wd"])
    og = O.Gpt(**C5)
    O.set_threads(min(16, os.cpu_count() or 1))
    n = C5["B"] * C5["T"]
    try:
        for t in (1, 2, 3):
            x, y = O.rand_tokens(3 << 24 | t, n, C5["V"]), O.rand_tokens(5 << 24 | t, n, C5["V"])
            hx, hy = rt.tensor(x), rt.tensor(y)
            hl = rt.L.malus_gpt_step(g, hx, hy, t)
            lg = rt.numpy(hl)[0]
            rt.free(hl, hx, hy)
            lo = og.step(x, y, t)
            print(f"C5 step {t}: gpu {lg:.7f} oracle {lo:.7f} rel {abs(lg - lo) / lo:.2e}")
            assert abs(lg - lo) <= 1e-5 * lo, (t, lg, lo)
        # Adam's first steps move each parameter by about lr * sign(gradient),
        # so a gradient within rounding of zero may step either way; the
        # rest agree to f32 rounding.
        diffs = np.concatenate([np.abs(rt.numpy(rt.L.malus_gpt_param(g, i)).ravel() - og.param(i))
                                for i in range(og.nparams)])
        frac = float(np.mean(diffs > 1e-5))
        print(f"C5 parameters after 3 steps: max |diff| {diffs.max():.2e}, fraction above 1e-5: {frac:.2e}")
        assert frac <= 1e-3
    finally:
        rt.L.malus_gpt_free(g)
        rt.L.tape_reset()
