"""bf16 storage under autocast (docs/adr/0037-bf16-autocast.md:8 and :30):
the stdlib's f32 <-> bf16 conversion, GEMMs whose operands are stored in
bf16, and the model's storage policy (the layernorm-scale outputs, gelu(h)
and the GELU VJP's dh kept in bf16).

Parity pins:
- the conversion is torch's float32 -> bfloat16 conversion (round to nearest
  even, NaN kept, infinities and subnormals as IEEE rounds them), and bf16 ->
  f32 returns the same values;
- under autocast a GEMM rounds f32 operands to bf16 before the MFMA, so the
  same GEMM on a bf16-stored copy of an operand sees identical values and
  must return identical bits, for every form (NN, NT, TN, split K), tile
  and edge shape the kernels take;
- the model under autocast with bf16 storage must equal, bit for bit, the
  same model with every activation stored in f32 (losses, parameters and
  both Adam moments over several steps), and hold less memory."""
import ctypes as C

import numpy as np
import pytest
import torch

import malus_amd as M
from oracle import oracle as O

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(53)
OPT = dict(lr=1e-3, b1=0.9, b2=0.99, eps=1e-8, wd=0.1)


def rand(*shape):
    return RNG.uniform(-1.0, 1.0, size=shape).astype(np.float32)


def run(rt, h):
    assert h, rt.last_error()
    out = rt.numpy(h)
    rt.free(h)
    return out


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_cast_is_torchs_bfloat16_conversion(rt):
    specials = np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 3.4e38, -3.4e38, 1e-45, -1e-45, 1.17e-38,
                         1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, 1.0 + 2.0 ** -8 + 2.0 ** -20, 65504.0, 0.1, 1.0 / 3.0],
                        np.float32)
    u = RNG.integers(0, 2 ** 32, 100_000, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([specials, u.view(np.float32), rand(4096) * 1e3])
    hx = rt.tensor(x)
    h16 = rt.L.malus_std_cast(hx, M.BF16)
    assert h16, rt.last_error()
    assert rt.L.malus_tensor_dtype(h16) == M.BF16
    got = rt.numpy(h16)
    want = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(bits(got)[~nan], bits(want)[~nan])
    back = run(rt, rt.L.malus_std_cast(h16, M.F32))
    assert np.array_equal(bits(back)[~nan], bits(got)[~nan]) and np.isnan(back[nan]).all()
    finite = np.isfinite(x) & (np.abs(x) < 3e38)
    assert np.array_equal(bits(got)[finite], bits(O.bf16_round(x[finite])))
    rt.free(hx, h16)


# (M, K, N) of C = A @ B; the dA / dB forms use the same three sizes (M % 16 ==
# 0 and N % 16 == 0: each is the K of one form; edge tiles in every dimension)
GEMM_SHAPES = [(512, 384, 1536), (1008, 384, 1536), (528, 1536, 384), (4096, 384, 1152), (96, 16, 208)]


# name: (entry point, operands uploaded in bf16); a [M, K], b [K, N], d [M, N]
FORMS = {
    "NN A16": ("tensor_matmul", "a"),               # C = a @ b
    "NN B16": ("tensor_matmul", "b"),
    "NN A16 B16": ("tensor_matmul", "ab"),
    "NT A16": ("malus_std_matmul_bwd_a", "d"),      # dA = d @ b^T
    "NT B16": ("malus_std_matmul_bwd_a", "b"),
    "NT A16 B16": ("malus_std_matmul_bwd_a", "db"),
    "TN A16": ("malus_std_matmul_bwd_b", "a"),      # dB = a^T @ d
    "TN A16 B16": ("malus_std_matmul_bwd_b", "ad"),
}


def _gemm(rt, entry, a, b, d, bf16=""):
    h = {k: rt.bf16(v) if k in bf16 else rt.tensor(v) for k, v in (("a", a), ("b", b), ("d", d))}
    try:
        fn = getattr(rt.L, entry)
        return run(rt, fn(h["a"], h["b"]) if entry == "tensor_matmul" else fn(h["a"], h["b"], h["d"]))
    finally:
        rt.free(*h.values())


def _check_forms(rt, a, b, d, what):
    with M.autocast():
        for name, (entry, bf16) in FORMS.items():
            got, want = _gemm(rt, entry, a, b, d, bf16), _gemm(rt, entry, a, b, d)
            assert np.array_equal(bits(got), bits(want)), f"{name} {what}"


@pytest.mark.parametrize("shape", GEMM_SHAPES, ids=[f"{m}x{k}x{n}" for m, k, n in GEMM_SHAPES])
def test_bf16_operand_gemms_equal_f32_storage(rt, shape):
    m, k, n = shape
    a, b, d = rand(m, k), rand(k, n), rand(m, n)
    _check_forms(rt, a, b, d, shape)
    # and the value is the f32 sum of the bf16-rounded operands' products
    ref = O.bf16_round(a).astype(np.float64) @ O.bf16_round(b).astype(np.float64)
    with M.autocast():
        c = _gemm(rt, "tensor_matmul", a, b, d, "a")
    assert np.abs(c - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())


@pytest.mark.parametrize("tile", [(2, 3), (2, 2), (2, 1), (1, 2), (1, 1)])
def test_bf16_operand_gemms_every_tile(rt, tile):
    a, b, d = rand(1008, 384), rand(384, 1536), rand(1008, 1536)
    assert rt.L.malus_gemm_set_tile(*tile)
    try:
        _check_forms(rt, a, b, d, f"tile {tile}")
    finally:
        rt.L.malus_gemm_set_tile(0, 0)


def test_bf16_operand_weight_gradient_split_k(rt):
    """dW = x^T dh at the C5 MLP's shape and token count: K = 16,384 splits
    across workgroups (f32 partials, summed in split order)."""
    x, w, dh = rand(16384, 384), rand(384, 1536), rand(16384, 1536)
    with M.autocast():
        got = _gemm(rt, "malus_std_matmul_bwd_b", x, w, dh, "ad")
        want = _gemm(rt, "malus_std_matmul_bwd_b", x, w, dh)
    assert np.array_equal(bits(got), bits(want))


def test_bf16_operands_the_kernels_cannot_take_are_errors(rt):
    rt.L.malus_set_abort_on_error(0)
    try:
        with M.autocast():
            # K = 7: no LDS-DMA kernel, so no bf16 operand path
            h = rt.L.tensor_matmul(rt.bf16(rand(5, 7)), rt.tensor(rand(7, 3)))
            assert h == 0 and "LDS-DMA" in rt.last_error()
            rt.L.malus_clear_error()
            # a weight gradient from an f32 activation and a bf16 gradient has no instance
            h = rt.L.malus_std_matmul_bwd_b(rt.tensor(rand(64, 64)), rt.tensor(rand(64, 64)), rt.bf16(rand(64, 64)))
            assert h == 0 and "bf16 storage mask" in rt.last_error()
            rt.L.malus_clear_error()
        # elementwise ops take f32 only
        h = rt.L.malus_std_gelu_fwd(rt.bf16(rand(8)))
        assert h == 0 and "f32" in rt.last_error()
        rt.L.malus_clear_error()
        h = rt.L.malus_std_cast(rt.tensor(np.arange(4, dtype=np.int32)), M.BF16)
        assert h == 0 and "f32 and bf16" in rt.last_error()
        rt.L.malus_clear_error()
    finally:
        rt.L.malus_set_abort_on_error(1)


C5 = dict(V=65, T=256, C=384, H=6, L=6, B=64)


def _make(rt, cfg, bf16_act):
    rt.L.tape_reset()
    rt.L.malus_rng_set_counter(0)
    g = rt.L.malus_gpt_create(cfg["V"], cfg["T"], cfg["C"], cfg["H"], cfg["L"], cfg["B"], OPT["lr"], OPT["b1"],
                              OPT["b2"], OPT["eps"], OPT["wd"])
    rt.L.malus_gpt_set_bf16_activations(g, 1 if bf16_act else 0)
    return g


def _state(rt, g):
    out = []
    for i in range(rt.L.malus_gpt_nparams(g)):
        out.append(rt.numpy(rt.L.malus_gpt_param(g, i)))
        out.append(rt.numpy(rt.L.malus_gpt_moment(g, i, 0)))
        out.append(rt.numpy(rt.L.malus_gpt_moment(g, i, 1)))
    return out


def test_c5_bf16_activations_equal_f32_storage(rt):
    """The autocast C5 step with the storage policy on and off: the same
    bits after 3 steps, and the forward's saved activations take less
    memory with it on (the two layernorm outputs and gelu(h) of 6 layers
    at half size: 6 * (2 * 16384 * 384 + 16384 * 1536) * 2 bytes = 453 MB)."""
    n = C5["B"] * C5["T"]
    batches = [(O.rand_tokens((5 << 32) + 2 * n * k, n, C5["V"]), O.rand_tokens((5 << 32) + 2 * n * k + n, n, C5["V"]))
               for k in range(3)]
    runs, live = {}, {}
    with M.autocast():
        for on in (True, False):
            g = _make(rt, C5, on)
            hx, hy = rt.tensor(batches[0][0]), rt.tensor(batches[0][1])
            base = rt.L.malus_pool_live_bytes()
            loss = rt.L.malus_gpt_forward_loss(g, hx, hy)
            live[on] = rt.L.malus_pool_live_bytes() - base
            rt.free(loss)
            rt.L.tape_reset()
            losses = []
            for k, (x, y) in enumerate(batches):
                hx2, hy2 = rt.tensor(x), rt.tensor(y)
                hl = rt.L.malus_gpt_step(g, hx2, hy2, k + 1)
                losses.append(rt.numpy(hl)[0])
                rt.free(hl, hx2, hy2)
            runs[on] = (losses, _state(rt, g))
            rt.free(hx, hy)
            rt.L.malus_gpt_free(g)
            rt.L.tape_reset()
    print(f"C5 autocast losses: bf16 storage {runs[True][0]}, f32 storage {runs[False][0]}; "
          f"forward live bytes {live[True] / 1e6:.0f} MB vs {live[False] / 1e6:.0f} MB")
    assert runs[True][0] == runs[False][0]
    for i, (a, b) in enumerate(zip(runs[True][1], runs[False][1])):
        assert np.array_equal(bits(a), bits(b)), f"state tensor {i} differs"
    assert live[False] - live[True] >= 0.9 * 6 * (2 * n * 384 + n * 1536) * 2


C4 = dict(V=65, T=64, C=128, H=4, L=4, B=32)


@pytest.mark.parametrize("attention", [1, 2], ids=["flash", "rows"])
def test_c4_bf16_activations_equal_f32_storage(rt, attention):
    """The policy at C4 (head size 32) under both fused attentions: with the
    row-register attention q, k, v stay f32 while the layernorm outputs,
    gelu(h), dh and the weight copies are bf16 (the head-projection GEMMs then
    take a bf16 A with an f32 C, and their dx a bf16 weight with f32 dq).
    3 steps with the policy on equal the steps with it off, bit for bit."""
    n = C4["B"] * C4["T"]
    batches = [(O.rand_tokens((7 << 32) + 2 * n * k, n, C4["V"]), O.rand_tokens((7 << 32) + 2 * n * k + n, n, C4["V"]))
               for k in range(3)]
    runs = {}
    with M.autocast():
        for on in (True, False):
            g = _make(rt, C4, on)
            assert rt.L.malus_gpt_set_attention(g, attention) == 0
            losses = []
            for k, (x, y) in enumerate(batches):
                hx, hy = rt.tensor(x), rt.tensor(y)
                hl = rt.L.malus_gpt_step(g, hx, hy, k + 1)
                losses.append(rt.numpy(hl)[0])
                rt.free(hl, hx, hy)
            runs[on] = (losses, _state(rt, g))
            rt.L.malus_gpt_free(g)
            rt.L.tape_reset()
    assert runs[True][0] == runs[False][0]
    for i, (a, b) in enumerate(zip(runs[True][1], runs[False][1])):
        assert np.array_equal(bits(a), bits(b)), f"state tensor {i} differs"
