"""The f32 GEMM's two product paths through the C ABI
(malus_gemm_set_f32_split): split (default; each f32 operand value as
three exact bf16 pieces, six piece products on the bf16 MFMA, f32
accumulation) and the FP32 MFMA.  The matmul it serves is
crates/malus-runtime/src/metal.rs:802-962 (tensor_matmul, f32 in, f32 out).

What pins the split path (beyond the oracle parity every matmul, model and
trajectory test already checks at 1e-5 normwise / 1e-3 over 200 steps):
  * the pieces are exact: X @ I and I @ X reproduce X bit for bit over a
    2^+-30 range of magnitudes, in every operand orientation;
  * its error against float64 is no larger than the FP32 MFMA's on the C5
    shapes (NN, NT, TN with K up to 4096 tokens);
  * non-finite operands reach exactly the outputs a GEMM's data flow says
    they reach, and no other output changes;
  * the fused attention kernels keep the composed ops' bits on both paths.
"""
import numpy as np
import pytest

from tests.helpers import assert_bitexact

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(4321)


class split_mode:
    """with split_mode(rt, on): the GEMM product path for the block."""

    def __init__(self, rt, on):
        self.L, self.on = rt.L, on

    def __enter__(self):
        self.prev = self.L.malus_gemm_set_f32_split(1 if self.on else 0)

    def __exit__(self, *exc):
        self.L.malus_gemm_set_f32_split(self.prev)


def matmul(rt, a, b, form="nn"):
    """C = a @ b (nn), a @ b.T (nt: b stored [N, K]) or a.T @ b (tn: a stored
    [K, M]) through tensor_matmul and the matmul VJP entry points."""
    L = rt.L
    ha, hb = rt.tensor(a), rt.tensor(b)
    if form == "nn":
        h = L.tensor_matmul(ha, hb)
        hz = 0
    elif form == "nt":  # dA = dout @ B^T with dout = a [M, K], B = b [N, K]
        hz = rt.tensor(np.zeros((a.shape[0], b.shape[0]), np.float32))
        h = L.malus_std_matmul_bwd_a(hz, hb, ha)
    else:  # dB = A^T @ dout with A = a [K, M], dout = b [K, N]
        hz = rt.tensor(np.zeros((a.shape[1], b.shape[1]), np.float32))
        h = L.malus_std_matmul_bwd_b(ha, hz, hb)
    assert h, rt.last_error()
    out = rt.numpy(h)
    rt.free(h, ha, hb, hz)
    return out


def ref64(a, b, form):
    a, b = a.astype(np.float64), b.astype(np.float64)
    return a @ b if form == "nn" else a @ b.T if form == "nt" else a.T @ b


@pytest.mark.parametrize("split", [True, False], ids=["split", "fp32"])
def test_identity_products_are_exact(rt, split):
    # one 16-deep slab's pieces sum back to each value exactly, so a product
    # with the identity returns the other operand bit for bit, for values
    # from 2^-30 to 2^30 times N(0, 1) and both operand roles
    x = (RNG.standard_normal((1024, 256)) * np.exp2(RNG.integers(-30, 31, (1024, 256)))).astype(np.float32)
    eye = np.eye(256, dtype=np.float32)
    with split_mode(rt, split):
        assert_bitexact(matmul(rt, x, eye), x, "X @ I")
        assert_bitexact(matmul(rt, eye, np.ascontiguousarray(x.T)), x.T, "I @ X^T")
        assert_bitexact(matmul(rt, x, eye, "nt"), x, "X @ I^T")
        assert_bitexact(matmul(rt, eye, x.T.copy(), "tn"), x.T, "I^T @ X^T")


# The C5 shapes with the token count cut to 4096 (K = tokens for TN)
SHAPES = [("nn", 4096, 384, 384), ("nn", 4096, 384, 1536), ("nn", 4096, 1536, 384),
          ("nt", 4096, 384, 1536), ("nt", 4096, 1536, 384),
          ("tn", 4096, 384, 384), ("tn", 4096, 384, 1536), ("tn", 4096, 1536, 384)]


@pytest.mark.parametrize("form,t,k,n", SHAPES, ids=[f"{f}-{k}x{n}" for f, _, k, n in SHAPES])
def test_split_error_vs_float64_no_larger_than_fp32_mfma(rt, form, t, k, n):
    # activations N(0, 1) against weights N(0, 0.02) (nn, nt), activations
    # against gradients (tn)
    if form == "nn":
        a, b = RNG.standard_normal((t, k)), RNG.standard_normal((k, n)) * 0.02
    elif form == "nt":
        a, b = RNG.standard_normal((t, k)), RNG.standard_normal((n, k)) * 0.02
    else:
        a, b = RNG.standard_normal((t, k)), RNG.standard_normal((t, n)) * 1e-3
    a, b = a.astype(np.float32), b.astype(np.float32)
    want = ref64(a, b, form)
    scale = np.abs(want).max()
    errs = {}
    for split in (True, False):
        with split_mode(rt, split):
            got = matmul(rt, a, b, form).astype(np.float64)
        d = np.abs(got - want)
        errs[split] = (d.max() / scale, np.sqrt(np.mean(d * d) / np.mean(want * want)))
    (mx_s, rms_s), (mx_f, rms_f) = errs[True], errs[False]
    print(f"{form} {t}x{k}x{n}: split max {mx_s:.2e} rms {rms_s:.2e} | fp32 max {mx_f:.2e} rms {rms_f:.2e}")
    assert mx_s <= 1e-5 and rms_s <= 1e-6
    # no larger than the FP32 MFMA's error: the rms within 10 %, the max
    # (one extreme element of one draw) within 50 %
    assert mx_s <= 1.5 * mx_f and rms_s <= 1.1 * rms_f, errs


@pytest.mark.parametrize("split", [True, False], ids=["split", "fp32"])
def test_nonfinite_operands_reach_only_their_outputs(rt, split):
    # An inf in A row r (or B column j) makes row r (column j) non-finite --
    # NaN on the split path, where the inf's residual inf - inf is NaN -- and
    # leaves every other output bit-identical to the product without it
    # (rows and columns of a GEMM are independent).
    a = RNG.uniform(-1, 1, (256, 64)).astype(np.float32)
    b = RNG.uniform(-1, 1, (64, 160)).astype(np.float32)
    with split_mode(rt, split):
        clean = matmul(rt, a, b)
        a2 = a.copy()
        a2[5, 7] = np.inf
        got = matmul(rt, a2, b)
        assert not np.isfinite(got[5]).any()
        rows = np.arange(256) != 5
        assert_bitexact(got[rows], clean[rows], "rows without the inf")
        b2 = b.copy()
        b2[9, 33] = -np.inf
        got = matmul(rt, a, b2)
        assert not np.isfinite(got[:, 33]).any()
        cols = np.arange(160) != 33
        assert_bitexact(got[:, cols], clean[:, cols], "columns without the inf")


@pytest.mark.parametrize("t,hs,causal", [(256, 64, 1), (64, 32, 0)])
def test_fused_attention_equals_composed_ops_on_fp32_mfma(rt, t, hs, causal):
    # the same bit-identity the default-path tests check, with every GEMM and
    # the fused kernels on the FP32 MFMA
    from tests import test_kernels_gpu as K

    with split_mode(rt, False):
        K.test_attn_fwd_equals_composed_ops(rt, t, hs, causal)
        K.test_attn_bwd_all_equals_composed_ops(rt, t, hs, causal, 5)


def test_model_fusions_equal_separate_ops_on_fp32_mfma(rt):
    from tests import test_models_gpu as TM

    with split_mode(rt, False):
        TM.test_gpt_fusions_equal_separate_ops(rt, dict(V=65, T=64, C=64, H=4, L=2, B=4))
        TM.test_gpt_fusions_equal_separate_ops(rt, dict(V=65, T=256, C=128, H=2, L=1, B=2))


def test_set_f32_split_returns_previous(rt):
    L = rt.L
    prev = L.malus_gemm_set_f32_split(0)
    try:
        assert L.malus_gemm_set_f32_split(1) == 0
        assert L.malus_gemm_set_f32_split(1) == 1
    finally:
        L.malus_gemm_set_f32_split(prev)


def test_weight_split_copies_give_the_same_steps(rt):
    # With split products the model's forward GEMMs read B from split copies
    # of the block weights (three bf16 planes, refreshed each forward)
    # instead of splitting the weights themselves: three steps
    # with the copies (malus_gpt_set_bf16_activations 1, the default) equal
    # three without, bit for bit (losses, parameters and both moments).
    from tests.test_models_gpu import GpuGpt, tokens

    cfg = dict(V=65, T=64, C=128, H=4, L=2, B=8)
    x, y = tokens(cfg, 777)
    out = []
    with split_mode(rt, True):
        for copies in (1, 0):
            g = GpuGpt(rt, cfg)
            try:
                rt.L.malus_gpt_set_bf16_activations(g.g, copies)
                losses = [g.step(x, y, t) for t in (1, 2, 3)]
                state = [g.param(i) for i in range(8 * cfg["L"] + 4)]
                state += [rt.numpy(rt.L.malus_gpt_moment(g.g, i, m)).ravel() for m in (0, 1)
                          for i in range(8 * cfg["L"] + 4)]
            finally:
                g.close()
            out.append((losses, state))
    assert out[0][0] == out[1][0]
    for i, (u, v) in enumerate(zip(out[0][1], out[1][1])):
        np.testing.assert_array_equal(u, v, err_msg=f"state {i}")
