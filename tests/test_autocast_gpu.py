"""bf16 autocast (docs/adr/0037-bf16-autocast.md:5-12: matmuls in bf16,
f32 master weights, f32 reductions) through the C ABI.

GEMM parity pin: under autocast each product is the f32 accumulation of
the bf16-rounded operands, so the oracle's f32 matmul of O.bf16_round(a) and
O.bf16_round(b) is the reference result; the tolerance is the f32 one
(normwise 1e-5: a bf16 x bf16 product is exact in f32, only the summation
order differs).  The same result is checked to differ from the unrounded
f32 product (the scope took effect) and the f32 path to be unchanged after
the scope ends.

Model: the ADR's success bar is convergence parity with the f32 run; the
C4 step under autocast is compared with the f32 oracle (loss within 1e-2
relative, gradients normwise within 5e-2: bf16 operands carry 2^-9 relative
error per element), and a 100-step run on a learnable corpus must stay
within 2% of the f32 oracle's loss at every 10th step."""
import numpy as np
import pytest

import malus_amd as M
from oracle import oracle as O
from tests.helpers import assert_normwise, normwise_err

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(37)
C4 = dict(V=65, T=64, C=128, H=4, L=4, B=32)
OPT = dict(lr=1e-3, b1=0.9, b2=0.99, eps=1e-8, wd=0.1)


def rand(*shape):
    return RNG.uniform(-1.0, 1.0, size=shape).astype(np.float32)


def run(rt, h):
    out = rt.numpy(h)
    rt.free(h)
    return out


def bt(x):
    return O.permute(x, (0, 2, 1)) if x.ndim == 3 else O.permute(x, (1, 0))


MM_SHAPES = [((2, 3), (3, 2)), ((65, 127), (127, 129)), ((128, 128), (128, 128)), ((300, 384), (384, 65)),
             ((8, 64, 32), (8, 32, 48)), ((3, 5, 7), (7, 9)), ((384, 1024), (1024, 384)), ((16384, 4), (4, 8)),
             ((1024, 384), (384, 1536))]


@pytest.mark.parametrize("sa,sb", MM_SHAPES)
def test_autocast_matmul_and_vjps_are_f32_sums_of_bf16_products(rt, sa, sb):
    a, b = rand(*sa), rand(*sb)
    ra, rb = O.bf16_round(a), O.bf16_round(b)
    ha, hb = rt.tensor(a), rt.tensor(b)
    with M.autocast():
        c = run(rt, rt.L.tensor_matmul(ha, hb))
        d = rand(*c.shape)
        rd = O.bf16_round(d)
        hd = rt.tensor(d)
        da = run(rt, rt.L.malus_std_matmul_bwd_a(ha, hb, hd))
        db = run(rt, rt.L.malus_std_matmul_bwd_b(ha, hb, hd))
    assert_normwise(c, O.matmul(ra, rb), 1e-5, f"autocast matmul {sa}@{sb}")
    assert_normwise(da, O.matmul(rd, bt(rb)).reshape(a.shape), 1e-5, "autocast dA")
    if a.ndim == 3 and b.ndim == 2:
        wb = O.reduce_axis(O.R_SUM, O.matmul(bt(ra), rd), 0)
    else:
        wb = O.matmul(bt(ra), rd)
    assert_normwise(db, wb.reshape(b.shape), 1e-5, "autocast dB")
    if c.size >= 64:
        # the operands were rounded: the f32 product is farther away than the f32 tolerance
        assert normwise_err(c, O.matmul(a, b)) > 1e-4
    rt.free(ha, hb, hd)


@pytest.mark.parametrize("tile", [(2, 3), (2, 2), (2, 1), (1, 2), (1, 1)])
@pytest.mark.parametrize("dma", [1, 0])
def test_autocast_every_tile_and_staging_path(rt, tile, dma):
    a, b = rand(700, 384), rand(384, 520)
    want = O.matmul(O.bf16_round(a), O.bf16_round(b))
    ha, hb = rt.tensor(a), rt.tensor(b)
    rt.L.malus_gemm_set_tile(*tile)
    rt.L.malus_gemm_set_dma(dma)
    try:
        with M.autocast():
            got = run(rt, rt.L.tensor_matmul(ha, hb))
    finally:
        rt.L.malus_gemm_set_tile(0, 0)
        rt.L.malus_gemm_set_dma(1)
    assert_normwise(got, want, 1e-5, f"tile {tile} dma {dma}")
    rt.free(ha, hb)


def test_autocast_split_k_weight_grad(rt):
    # dW of a C5 projection ([384, 16384] @ [16384, 384], the split-K path)
    x, d, w = rand(16384, 384), rand(16384, 384), rand(384, 384)
    hx, hd, hw = rt.tensor(x), rt.tensor(d), rt.tensor(w)
    with M.autocast():
        got = run(rt, rt.L.malus_std_matmul_bwd_b(hx, hw, hd))
    O.set_threads(8)
    assert_normwise(got, O.matmul(O.bf16_round(x).T.copy(), O.bf16_round(d)), 1e-5, "autocast split-K dW")
    rt.free(hx, hd, hw)


def test_autocast_scope_restores_f32(rt):
    a, b = rand(256, 192), rand(192, 320)
    ha, hb = rt.tensor(a), rt.tensor(b)
    before = run(rt, rt.L.tensor_matmul(ha, hb))
    with M.autocast():
        inside = run(rt, rt.L.tensor_matmul(ha, hb))
        with M.autocast(False):
            nested_off = run(rt, rt.L.tensor_matmul(ha, hb))
        inside2 = run(rt, rt.L.tensor_matmul(ha, hb))
    after = run(rt, rt.L.tensor_matmul(ha, hb))
    assert rt.L.malus_autocast(0) == 0  # the scope left it off
    np.testing.assert_array_equal(before, after)
    np.testing.assert_array_equal(before, nested_off)
    np.testing.assert_array_equal(inside, inside2)
    assert not np.array_equal(before, inside)
    assert_normwise(before, O.matmul(a, b), 1e-5, "f32 outside the scope")
    rt.free(ha, hb)


# ------------------------------------------------------------------- model
class Gpt:
    def __init__(self, rt, cfg):
        self.rt = rt
        rt.L.tape_reset()
        rt.L.malus_rng_set_counter(0)
        self.g = rt.L.malus_gpt_create(cfg["V"], cfg["T"], cfg["C"], cfg["H"], cfg["L"], cfg["B"], OPT["lr"],
                                       OPT["b1"], OPT["b2"], OPT["eps"], OPT["wd"])
        self.n = 8 * cfg["L"] + 4

    def close(self):
        self.rt.L.malus_gpt_free(self.g)
        self.rt.L.tape_reset()

    def grad(self, i):
        g = self.rt.L.tape_get_grad(self.rt.L.malus_gpt_param(self.g, i))
        out = self.rt.numpy(g).ravel()
        self.rt.free(g)
        return out

    def loss_and_grads(self, x, y):
        rt = self.rt
        hx, hy = rt.tensor(x), rt.tensor(y)
        rt.L.malus_gpt_zero_grad(self.g)
        loss = rt.L.malus_gpt_forward_loss(self.g, hx, hy)
        rt.L.backward(loss)
        v = rt.numpy(loss)[0]
        rt.free(hx, hy, loss)
        return v

    def step(self, x, y, t):
        rt = self.rt
        hx, hy = rt.tensor(x), rt.tensor(y)
        loss = rt.L.malus_gpt_step(self.g, hx, hy, t)
        v = rt.numpy(loss)[0]
        rt.free(hx, hy, loss)
        return v


def corpus(n, vocab, seed=11):
    """A learnable token stream: a fixed 97-token phrase repeated, with a
    tenth of the positions replaced by random tokens."""
    rng = np.random.default_rng(seed)
    phrase = rng.integers(0, vocab, 97)
    data = np.resize(phrase, n)
    noise = rng.random(n) < 0.1
    data[noise] = rng.integers(0, vocab, int(noise.sum()))
    return data.astype(np.int32)


def batch(data, cfg, step):
    rng = np.random.default_rng(1000 + step)
    starts = rng.integers(0, len(data) - cfg["T"] - 1, cfg["B"])
    x = np.concatenate([data[s:s + cfg["T"]] for s in starts]).astype(np.int32)
    y = np.concatenate([data[s + 1:s + cfg["T"] + 1] for s in starts]).astype(np.int32)
    return x, y


def test_autocast_c4_step_vs_f32_oracle(rt):
    x, y = batch(corpus(20000, C4["V"]), C4, 0)
    og = O.Gpt(**C4)
    O.set_threads(16)
    wloss = og.loss_and_grads(x, y)
    g = Gpt(rt, C4)
    try:
        with M.autocast():
            loss = g.loss_and_grads(x, y)
        errs = [normwise_err(g.grad(i), og.grad(i)) for i in range(g.n)]
    finally:
        g.close()
    print(f"autocast C4: loss {loss:.6f} vs f32 oracle {wloss:.6f}; worst gradient error {max(errs):.2e}")
    assert abs(loss - wloss) <= 1e-2 * abs(wloss)
    assert max(errs) <= 5e-2
    # and not the f32 result: the operands were rounded
    assert abs(loss - wloss) > 0 or max(errs) > 1e-4


def test_autocast_c4_convergence_parity(rt):
    data = corpus(20000, C4["V"])
    og = O.Gpt(**C4)
    O.set_threads(16)
    g = Gpt(rt, C4)
    worst = 0.0
    try:
        with M.autocast():
            for t in range(1, 101):
                x, y = batch(data, C4, t)
                lg = g.step(x, y, t)
                lo = og.step(x, y, t)
                if t % 10 == 0:
                    worst = max(worst, abs(lg - lo) / lo)
                    print(f"step {t}: autocast {lg:.4f} f32 oracle {lo:.4f}")
                    assert abs(lg - lo) <= 0.02 * lo, f"step {t}: {lg} vs {lo}"
    finally:
        g.close()
    assert lo < 0.5 * np.log(C4["V"])  # the corpus was learned (4.17 -> about 1.6)
    print(f"autocast C4 100 steps: worst relative loss difference {worst:.2e}")
