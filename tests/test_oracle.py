"""Pins the CPU oracle before it is trusted as the checker.

Each oracle function is checked against something it does not share code
with: the reference's own known answers (crates/malus-runtime/src/tests.rs,
crates/malus-codegen-cpu/tests/metal_integration.rs, README.md), the
published Random123 Philox vectors, numpy/float64 closed forms, adjoint
identities, and central finite differences for every VJP.  CPU only.
"""
import numpy as np
import pytest

from oracle import oracle as O

from tests.helpers import KATS, assert_bitexact

RNG = np.random.default_rng(7)


def r(*s, lo=-1, hi=1):
    return RNG.uniform(lo, hi, size=s).astype(np.float32)


# --------------------------------------------------------------------- RNG
@pytest.mark.parametrize("kat", KATS["philox4x32_10"], ids=lambda k: "%08x" % k["ctr"][0])
def test_philox_random123_kat_vectors(kat):
    assert O.philox(kat["ctr"], kat["key"]) == kat["out"]


def test_randn_is_box_muller_of_philox_pairs():
    # metal.rs:1727-1738 recomputed in numpy float64 from raw Philox words
    call = 12
    z = O.randn(call, (7,))
    for k in range(4):
        w = O.philox([k, 0, 0, 0], [call, 0])
        u1, u2 = (w[0] + 0.5) / 2**32, (w[1] + 0.5) / 2**32
        mag = np.sqrt(-2.0 * np.log(u1))
        assert z[2 * k] == np.float32(mag * np.cos(2 * np.pi * u2))
        if 2 * k + 1 < 7:
            assert z[2 * k + 1] == np.float32(mag * np.sin(2 * np.pi * u2))


def test_randn_statistics_and_call_keying():
    z = O.randn(3, (200000,))
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01
    assert np.array_equal(O.randn(3, (10,)), z[:10])  # prefix-stable per call index
    assert not np.array_equal(O.randn(4, (10,)), z[:10])


def test_rand_uniform_and_int():
    w = O.philox([0, 0, 0, 0], [9, 0])
    assert O.lib().or_rand_uniform(9) == np.float32(w[0] / 2**32)
    w1 = O.philox([1, 0, 0, 0], [9, 0])
    assert O.lib().or_rand_int(9, 65) == w1[0] % 65
    toks = O.rand_tokens(100, 5000, 65)
    assert toks.min() >= 0 and toks.max() < 65 and len(np.unique(toks)) == 65


# -------------------------------------------------------------- known answers
def f32(x):
    return np.array(x, np.float32)


def test_matmul_kats():
    for kat in KATS["matmul"]:
        assert np.array_equal(O.matmul(f32(kat["a"]), f32(kat["b"])), f32(kat["out"])), kat["source"]
    kat = KATS["add_matmul_add_chain"]
    a = f32(kat["a"])
    x = O.broadcast(O.ADD, a, a)
    y = O.matmul(x, x)
    assert np.array_equal(O.broadcast(O.ADD, y, y), f32(kat["out"])), kat["source"]


def test_broadcast_and_reduce_kats():
    ops = {"add": O.ADD, "sub": O.SUB}
    for kat in KATS["broadcast"]:
        got = O.broadcast(ops[kat["op"]], f32(kat["a"]), f32(kat["b"]))
        assert np.array_equal(got, f32(kat["out"])), kat["source"]
    rops = {"sum": O.R_SUM, "mean": O.R_MEAN, "max": O.R_MAX, "var": O.R_VAR}
    for kat in KATS["reduce"]:
        got = O.reduce_axis(rops[kat["op"]], f32(kat["x"]), kat["axis"], keepdim=bool(kat["keepdim"]))
        assert np.array_equal(got, f32(kat["out"])), kat["source"]
    # negative axis == positive axis (tests.rs:1087-1100)
    x = np.arange(12, dtype=np.float32).reshape(3, 4)
    assert np.array_equal(O.reduce_axis(O.R_SUM, x, -1), O.reduce_axis(O.R_SUM, x, 1))
    assert O.sum_all([1, 2, 3, 4]) == 10


def test_embedding_and_transpose_kats():
    for kat in KATS["embedding"]:
        assert np.array_equal(O.embedding(f32(kat["w"]), kat["idx"]), f32(kat["out"])), kat["source"]
    kat = KATS["embedding_bwd_counts"]
    g = O.embedding_bwd(np.ones((len(kat["idx"]), 3), np.float32), kat["idx"], kat["vocab"])
    assert g[:, 0].tolist() == kat["row_counts"] and np.all(g == g[:, :1])
    kat = KATS["transpose"]
    assert np.array_equal(O.permute(f32(kat["x"]), (1, 0)), f32(kat["out"])), kat["source"]


def test_softmax_layernorm_gelu_integration_kats():
    # the reference's inputs, compared with their inline formulas at the tolerance they use
    kat = KATS["integration_inputs"]
    tol = kat["tolerance"]
    x = f32(kat["softmax_x"])
    e = np.exp(x - x.max(1, keepdims=True))
    assert np.max(np.abs(O.softmax(x, 1) - e / e.sum(1, keepdims=True))) < tol
    y = f32(kat["layernorm_x"])
    ln, var = O.layernorm(y, 1)
    ref = (y - y.mean(1, keepdims=True)) / np.sqrt(y.var(1, keepdims=True) + 1e-5)
    assert np.max(np.abs(ln - ref)) < tol
    assert np.allclose(var.ravel(), y.var(1), rtol=tol)
    g = f32(kat["gelu_x"])
    inner = 0.7978845608028654 * (g + 0.044715 * g**3)
    assert np.max(np.abs(O.unary(O.GELU, g) - 0.5 * g * (1 + np.tanh(inner)))) < tol


def test_xor_readme_golden():
    kat = KATS["xor_readme"]
    loss, loss_at, preds, _ = O.xor_train()
    assert abs(loss - kat["loss"]) <= kat["rtol"] * kat["loss"]
    np.testing.assert_allclose(preds, kat["predictions"], rtol=kat["rtol"])
    assert loss_at[0] > 1.0 and np.all(np.diff(loss_at) < 0)


# ------------------------------------------------------------- closed forms
def test_elementwise_ops_are_single_ieee_ops():
    a, b = r(1000), r(1000, lo=0.5, hi=2)
    for op, f in [(O.ADD, np.add), (O.SUB, np.subtract), (O.MUL, np.multiply), (O.DIV, np.divide)]:
        assert np.array_equal(O.broadcast(op, a, b), f(a, b))
        assert np.array_equal(O.scalar_op(op, a, np.float32(0.3)), f(a, np.float32(0.3)))
        assert np.array_equal(O.scalar_op(op, b, np.float32(0.3), False), f(np.float32(0.3), b))
    # rank-mismatched sub computes b - a (broadcast_binop.ml:90-112)
    m = r(3, 5)
    assert np.array_equal(O.broadcast(O.SUB, a[:5], m), m - a[:5])
    assert np.array_equal(O.unary(O.RELU, a), np.maximum(a, 0))
    assert np.array_equal(O.unary(O.SQRT, b), np.sqrt(b))
    assert np.array_equal(O.unary(O.ABS, a), np.abs(a))


def test_transcendentals_within_libm_bounds_of_float64():
    # glibc documents expf/logf within 1 ulp and tanhf within 2 ulp
    x = r(20000, lo=-10, hi=10)
    for op, f, ulp in [(O.EXP, np.exp, 1), (O.TANH, np.tanh, 2)]:
        want = f(x.astype(np.float64)).astype(np.float32)
        got = O.unary(op, x)
        assert np.max(np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32))) <= ulp
    p = r(20000, lo=1e-3, hi=1e3)
    want = np.log(p.astype(np.float64)).astype(np.float32)
    assert np.max(np.abs(O.unary(O.LOG, p).view(np.int32).astype(np.int64) - want.view(np.int32))) <= 1


def test_matmul_within_sequential_error_bound():
    a, b = r(37, 300), r(300, 41)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    bound = 300 * np.finfo(np.float32).eps * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
    assert np.all(np.abs(O.matmul(a, b) - exact) <= bound)
    A, B = r(3, 5, 7), r(3, 7, 4)
    assert np.allclose(O.matmul(A, B), np.einsum("bmk,bkn->bmn", A.astype(np.float64), B), rtol=1e-5, atol=1e-6)
    assert np.allclose(O.matmul(A, B[0]), A.astype(np.float64) @ B[0], rtol=1e-5, atol=1e-6)


def _matmul_k_sequential(a, b):
    """metal.rs:698-800's summation, written as numpy float32 steps: every
    out[i,j] starts at 0.0 and adds the rounded product a[i,k]*b[k,j] for k
    ascending, each step rounded to f32 (separate multiply and add ufuncs)."""
    acc = np.zeros(a.shape[:-1] + (b.shape[-1],), np.float32)
    for kk in range(a.shape[-1]):
        acc = acc + a[..., kk:kk + 1] * b[..., kk:kk + 1, :]
    return acc


@pytest.mark.parametrize("m,k,n", [(13, 37, 70), (4, 5, 32), (1, 1, 1), (600, 9, 97), (8, 64, 31), (515, 3, 64)])
def test_matmul_is_the_k_sequential_sum_bit_for_bit(m, k, n):
    # the oracle's register tiles (4 x 32) and thread split (512-row chunks)
    # cover ragged rows and columns on both sides of every boundary
    a, b = r(m, k), r(k, n)
    for threads in (1, 8):
        O.set_threads(threads)
        assert_bitexact(O.matmul(a, b), _matmul_k_sequential(a, b), f"{m}x{k}x{n}, {threads} threads")
    A, B = r(3, m % 40 + 1, k), r(3, k, n)
    assert_bitexact(O.matmul(A, B), _matmul_k_sequential(A, B), "batched")
    assert_bitexact(O.matmul(A, B[1]), _matmul_k_sequential(A, B[1]), "3-D by 2-D")
    O.set_threads(1)


def test_bf16_round_is_torchs_bfloat16_conversion():
    # torch's f32 -> bfloat16 conversion rounds to nearest, ties to even
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 100000),
                        np.array([0.0, -0.0, 1.0, -2.5, 3e38, -3e38, 1e-40, 65504.0], np.float32)])
    # exact ties: the dropped 16 bits are 0x8000, with an even and an odd kept part
    tie_even = (np.arange(1000, dtype=np.uint32) * 2 << 16 | 0x8000) + 0x3F800000
    tie_odd = tie_even + 0x10000
    x = np.concatenate([x, tie_even.view(np.float32), tie_odd.view(np.float32), -tie_odd.view(np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    got = O.bf16_round(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # ties went to the even kept part: down for even, up for odd
    assert np.array_equal(O.bf16_round(tie_even.view(np.float32)).view(np.uint32), tie_even & 0xFFFF0000)
    assert np.array_equal(O.bf16_round(tie_odd.view(np.float32)).view(np.uint32), (tie_odd & 0xFFFF0000) + 0x10000)
    # idempotent, and within half a bf16 ulp (2^-9 relative)
    assert np.array_equal(O.bf16_round(got), got)
    nz = np.abs(x) > 1e-30
    assert np.all(np.abs(got[nz] - x[nz]) <= np.abs(x[nz]) * 2.0 ** -8)


def test_reductions_within_bound_and_shapes():
    x = r(13, 1000, 3)
    for axis in range(3):
        exact = x.astype(np.float64).sum(axis)
        n = x.shape[axis]
        bound = n * np.finfo(np.float32).eps * np.abs(x).astype(np.float64).sum(axis)
        assert np.all(np.abs(O.reduce_axis(O.R_SUM, x, axis) - exact) <= bound)
        assert np.array_equal(O.reduce_axis(O.R_MAX, x, axis), x.max(axis))
        assert np.allclose(O.reduce_axis(O.R_VAR, x, axis), x.astype(np.float64).var(axis), rtol=1e-4, atol=1e-6)


def test_softmax_layernorm_invariants():
    x = r(20, 300, lo=-5, hi=5)
    s = O.softmax(x, 1)
    assert np.allclose(s.sum(1), 1, atol=1e-5) and np.all(s > 0)
    assert np.allclose(O.softmax(x + 3.0, 1), s, atol=1e-6)  # shift invariance
    s0 = O.softmax(x, 0)
    assert np.allclose(s0.sum(0), 1, atol=1e-5)
    y, var = O.layernorm(x, 1)
    assert np.allclose(y.mean(1), 0, atol=1e-5) and np.allclose(y.var(1), 1, atol=1e-3)
    assert var.shape == (20, 1)


def test_cross_entropy_closed_form():
    logits = (RNG.standard_normal((50, 65)) * 2).astype(np.float32)
    t = RNG.integers(0, 65, 50).astype(np.int32)
    loss, probs = O.cross_entropy(logits, t)
    l64 = logits.astype(np.float64)
    lse = np.log(np.exp(l64 - l64.max(1, keepdims=True)).sum(1)) + l64.max(1)
    assert abs(loss - np.mean(lse - l64[np.arange(50), t])) < 1e-5
    g = O.cross_entropy_bwd(probs, t, 1.0)
    assert np.allclose(g.sum(1), 0, atol=1e-6)  # each row of softmax - onehot sums to 0


def test_causal_mask_and_permute_vs_numpy():
    assert np.array_equal(O.causal_mask(7), np.triu(np.full((7, 7), -1e9, np.float32), 1))
    x = r(2, 3, 4, 5)
    for perm in [(0, 2, 1, 3), (3, 2, 1, 0), (1, 0, 3, 2)]:
        assert np.array_equal(O.permute(x, perm), np.transpose(x, perm))


def test_adam_l2_matches_numpy_float32_expression():
    p, g, m, v = r(500), r(500), r(500) * 0.1, np.abs(r(500)) * 0.01
    lr, b1, b2, eps, wd = (np.float32(a) for a in (1e-3, 0.9, 0.99, 1e-8, 0.1))
    t = 3
    bc1 = np.float32(1) - np.float32(b1 ** np.float32(t))
    bc2 = np.float32(1) - np.float32(b2 ** np.float32(t))
    gg = g + p * wd
    mm = m * b1 + gg * (np.float32(1) - b1)
    vv = v * b2 + (gg * (np.float32(1) - b2)) * gg
    want = p - (mm / bc1 * lr) / (np.sqrt(vv / bc2) + eps)
    got, gm, gv = O.adam_l2(p, g, m, v, 1e-3, 0.9, 0.99, 1e-8, 0.1, 3)
    assert np.array_equal(gm, mm) and np.array_equal(gv, vv)
    assert np.max(np.abs(got - want)) <= 2 * np.max(np.spacing(np.abs(want)))  # powf vs numpy pow


def test_adam_l2_invariants():
    """Closed forms of the coupled-L2 Adam update that a dropped bias
    correction, a swapped beta or a misplaced weight-decay term would break."""
    p, g = r(400), r(400)
    z = np.zeros(400, np.float32)
    # t = 1 from zero moments: m_hat = g', v_hat = g'^2, so the step is lr * sign(g')
    # (up to eps) with g' = g + wd * p.
    for wd in (0.0, 0.1):
        got, gm, gv = O.adam_l2(p, g, z, z, 1e-3, 0.9, 0.99, 1e-8, wd, 1)
        gp = g.astype(np.float64) + wd * p.astype(np.float64)
        np.testing.assert_allclose(gm, 0.1 * gp, rtol=1e-6, atol=1e-9)
        np.testing.assert_allclose(gv, 0.01 * gp * gp, rtol=1e-5, atol=1e-12)
        step = p.astype(np.float64) - got
        keep = np.abs(gp) > 1e-3
        np.testing.assert_allclose(step[keep], 1e-3 * np.sign(gp[keep]), rtol=1e-4)
    # a constant gradient keeps m_hat = g and v_hat = g^2 at every t (bias
    # correction exactly undoes the zero start), so the second step is again
    # lr * sign(g); without the corrections it would be 0.19 / sqrt(0.0199) ~ 1.35x
    p1, m1, v1 = O.adam_l2(p, g, z, z, 1e-3, 0.9, 0.99, 1e-8, 0.0, 1)
    p2, m2, v2 = O.adam_l2(p1, g, m1, v1, 1e-3, 0.9, 0.99, 1e-8, 0.0, 2)
    keep = np.abs(g) > 1e-3
    np.testing.assert_allclose((p1 - p2)[keep].astype(np.float64), 1e-3 * np.sign(g[keep]), rtol=2e-3)
    np.testing.assert_allclose(m2, 0.19 * g.astype(np.float64), rtol=1e-5, atol=1e-9)
    # moments already at their fixed point (m = g', v = g'^2) stay there, and
    # for large t the step tends to lr * g' / (|g'| + eps)
    gp = g + np.float32(0.1) * p
    got, gm, gv = O.adam_l2(p, g, gp, gp * gp, 1e-3, 0.9, 0.99, 1e-8, 0.1, 5000)
    np.testing.assert_allclose(gm, gp, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(gv, gp * gp, rtol=1e-5, atol=1e-9)
    keep = np.abs(gp) > 1e-3
    np.testing.assert_allclose((p - got)[keep], 1e-3 * np.sign(gp[keep]), rtol=1e-3)
    # zero gradient and zero decay leave parameters and moments unchanged
    got, gm, gv = O.adam_l2(p, z, z, z, 1e-3, 0.9, 0.99, 1e-8, 0.0, 7)
    assert np.array_equal(got, p) and not gm.any() and not gv.any()


# ------------------------------------------------- adjoints / finite differences
def test_sum_to_shape_is_adjoint_of_broadcast():
    for xs, gs in [((5,), (4, 5)), ((1, 5), (3, 5)), ((1, 1), (6, 3, 4)), ((3, 1), (2, 3, 4))]:
        x, g = r(*xs).astype(np.float64), r(*gs).astype(np.float64)
        bx = np.broadcast_to(x, gs)
        lhs = float((bx * g).sum())
        rhs = float((x * O.sum_to_shape(g.astype(np.float32), xs)).sum())
        assert abs(lhs - rhs) < 1e-4 * (1 + abs(lhs))


def fd_check(f, x, grad, eps=1e-2, rtol=2e-2, n=40):
    """Central differences of scalar f (float64 accumulation) at n random coordinates."""
    x = x.astype(np.float32)
    idx = RNG.choice(x.size, size=min(n, x.size), replace=False)
    scale = max(np.max(np.abs(grad)), 1e-3)
    for i in idx:
        xp, xm = x.copy(), x.copy()
        xp.flat[i] += eps
        xm.flat[i] -= eps
        num = (f(xp) - f(xm)) / (float(xp.flat[i]) - float(xm.flat[i]))
        assert abs(num - grad.flat[i]) <= rtol * scale, f"coord {i}: numeric {num} vs analytic {grad.flat[i]}"


def wsum(w, y):
    return float((np.asarray(y, np.float64) * w).sum())


@pytest.mark.parametrize("op,lo,hi,use_out", [(O.SIGMOID, -3, 3, True), (O.TANH, -2, 2, True), (O.EXP, -2, 2, True),
                                              (O.SQRT, 0.5, 3, True), (O.LOG, 0.5, 3, False), (O.RELU, -2, 2, False),
                                              (O.ABS, -2, 2, False), (O.GELU, -3, 3, False)])
def test_unary_vjps_finite_differences(op, lo, hi, use_out):
    x = r(64, lo=lo, hi=hi)
    x = np.where(np.abs(x) < 0.05, 0.3, x).astype(np.float32)  # keep relu/abs away from the kink
    w = r(64).astype(np.float64)
    y = O.unary(op, x)
    if op == O.EXP:
        g = y * w.astype(np.float32)  # ExpBwd = dout * e (codegen-cpu/lib.rs:201)
    elif op == O.LOG:
        g = w.astype(np.float32) / x  # LogBwd = dout / x
    else:
        g = O.unary_bwd(op, y if use_out else x, w.astype(np.float32))
    fd_check(lambda z: wsum(w, O.unary(op, z)), x, g)


def test_softmax_vjp_finite_differences():
    x, w = r(6, 20, lo=-2, hi=2), r(6, 20).astype(np.float64)
    for axis in (0, 1):
        s = O.softmax(x, axis)
        fd_check(lambda z: wsum(w, O.softmax(z, axis)), x, O.softmax_bwd(s, w.astype(np.float32), axis))


def test_layernorm_vjp_finite_differences():
    x, w = r(5, 24, lo=-2, hi=2), r(5, 24).astype(np.float64)
    y, var = O.layernorm(x, 1)
    fd_check(lambda z: wsum(w, O.layernorm(z, 1)[0]), x, O.layernorm_bwd(y, var, w.astype(np.float32), 1), eps=5e-3)


def test_cross_entropy_vjp_finite_differences():
    x = r(8, 65, lo=-2, hi=2)
    t = RNG.integers(0, 65, 8).astype(np.int32)
    _, probs = O.cross_entropy(x, t)
    fd_check(lambda z: float(O.cross_entropy(z, t)[0]), x, O.cross_entropy_bwd(probs, t, 1.0), eps=1e-2)


def test_embedding_vjp_finite_differences():
    w, idx = r(6, 4), np.array([0, 3, 3, 5, 0, 0], np.int32)
    dout = r(6, 4).astype(np.float64)
    fd_check(lambda z: wsum(dout, O.embedding(z, idx)), w, O.embedding_bwd(dout.astype(np.float32), idx, 6))


def test_gpt_oracle_gradients_finite_differences():
    # the whole oracle backward (tape order, head fold/unfold, residual
    # accumulation, every VJP) against central differences of its own loss
    cfg = dict(V=11, T=8, C=16, H=4, L=2, B=2)
    g = O.Gpt(**cfg)
    n = cfg["B"] * cfg["T"]
    x, y = O.rand_tokens(50, n, cfg["V"]), O.rand_tokens(50 + n, n, cfg["V"])
    g.loss_and_grads(x, y)
    grads = [g.grad(i) for i in range(g.nparams)]
    h = O.Gpt(**cfg)
    # Directional derivative along a random unit direction mixed with the
    # gradient direction: large enough to move the f32 loss measurably, and a
    # transposed / mis-signed / mis-scaled gradient changes <g, d>.
    for pi in range(g.nparams):
        base = g.param(pi).astype(np.float64)
        gp = grads[pi].astype(np.float64)
        rnd = RNG.standard_normal(base.size)
        d = gp / np.linalg.norm(gp) + 0.5 * rnd / np.linalg.norm(rnd)
        d /= np.linalg.norm(d)
        eps = 0.05
        vals = []
        for s in (+eps, -eps):
            h.set_param(pi, (base + s * d).astype(np.float32))
            vals.append(float(h.loss_and_grads(x, y)))
        h.set_param(pi, base.astype(np.float32))
        num = (vals[0] - vals[1]) / (2 * eps)
        ana = float(gp @ d)
        assert abs(num - ana) <= 3e-2 * abs(ana) + 2e-5, (pi, num, ana)


@pytest.mark.parametrize("op", [O.R_SUM, O.R_MEAN, O.R_VAR])
@pytest.mark.parametrize("shape,axis", [((5, 24), 1), ((6, 4, 5), 1), ((7, 3), 0)])
def test_reduce_axis_vjps_finite_differences(op, shape, axis):
    x = r(*shape, lo=-2, hi=2)
    ysh = list(shape)
    ysh[axis] = 1
    w = r(*ysh).astype(np.float64)
    g = O.reduce_axis_bwd(op, x, w.astype(np.float32), axis)
    fd_check(lambda z: wsum(w, O.reduce_axis(op, z, axis, keepdim=True)), x, g, eps=5e-3)


def test_reduce_axis_vjps_closed_forms_and_max_ties():
    # mean: dout/N broadcast; var: dout * 2(x - mean)/N; max: every tied
    # maximum receives dout (reduce_bwd.ml:54-58), the others 0.
    x = np.array([[1, 3, 3, 2], [0, 5, -1, 5], [-4, -4, -4, -4]], np.float32)
    d = np.array([2, 3, 0.5], np.float32)
    np.testing.assert_array_equal(O.reduce_axis_bwd(O.R_MEAN, x, d, 1), np.repeat(d[:, None] * np.float32(0.25), 4, 1))
    y = O.reduce_axis(O.R_MAX, x, 1)
    np.testing.assert_array_equal(O.reduce_axis_bwd(O.R_MAX, x, d, 1, y),
                                  [[0, 2, 2, 0], [0, 3, 0, 3], [0.5, 0.5, 0.5, 0.5]])
    want_var = d[:, None].astype(np.float64) * 2 * (x - x.astype(np.float64).mean(1, keepdims=True)) / 4
    np.testing.assert_allclose(O.reduce_axis_bwd(O.R_VAR, x, d, 1), want_var, rtol=0, atol=1e-6)
    np.testing.assert_array_equal(O.reduce_axis_bwd(O.R_SUM, x, d, 0 + 1), np.repeat(d[:, None], 4, 1))
