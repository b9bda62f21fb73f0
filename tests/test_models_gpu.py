"""End-to-end parity of the workload drivers against the CPU oracle:
examples/xor.ml (C1), the toy char-nanoGPT (C4) and the Karpathy
char-nanoGPT (C5).  Loss trajectories: within 1e-3 relative (north star);
single-step gradients: normwise 3e-5 (per-op 1e-5 errors compound through
~40 dependent ops per block; measured worst 2.5e-6 at C4, 7.0e-6 at C5)."""
import ctypes as C
import os

import numpy as np
import pytest

import malus_amd as M
from oracle import oracle as O
from tests.emit_programs import SIGMOID_BACKWARD
from tests.helpers import normwise_err

pytestmark = pytest.mark.gpu

C4 = dict(V=65, T=64, C=128, H=4, L=4, B=32)
C5 = dict(V=65, T=256, C=384, H=6, L=6, B=64)
OPT = dict(lr=1e-3, b1=0.9, b2=0.99, eps=1e-8, wd=0.1)


def oracle_threads():
    return min(16, os.cpu_count() or 1)


def test_xor_10000_steps_vs_oracle(rt):
    # xor.ml's user kernel, lowered by the library's HIP emitter and compiled with hipRTC
    reg = M.compile_kernels(SIGMOID_BACKWARD)
    rt.L.malus_runtime_init(*reg.init_args())
    kid = reg.ids["sigmoid_backward"]
    assert not rt.L.malus_kernel_is_builtin(kid)
    loss_at = np.zeros(6, np.float32)
    preds = np.zeros(4, np.float32)
    params = np.zeros(33, np.float32)
    f = C.POINTER(C.c_float)
    loss = rt.L.malus_xor_run(10000, 1.5, kid, loss_at.ctypes.data_as(f), preds.ctypes.data_as(f),
                              params.ctypes.data_as(f))
    wl, wla, wp, wparams = O.xor_train(10000, 1.5)
    np.testing.assert_allclose(loss_at, wla, rtol=1e-3)
    np.testing.assert_allclose(preds, wp, rtol=1e-3)
    np.testing.assert_allclose(loss, wl, rtol=1e-3)
    # README.md:66-67 golden (Metal, fast-math): soft check
    np.testing.assert_allclose(preds, [0.0056860363, 0.99518234, 0.9939387, 0.005444207], rtol=1e-3)
    np.testing.assert_allclose(loss, 0.00012191984, rtol=1e-3)


class GpuGpt:
    def __init__(self, rt, cfg, rng_call_idx=0, fused=True, fused_forward=True):
        self.rt = rt
        self.cfg = cfg
        rt.L.tape_reset()
        rt.L.malus_rng_set_counter(rng_call_idx)
        self.g = rt.L.malus_gpt_create(cfg["V"], cfg["T"], cfg["C"], cfg["H"], cfg["L"], cfg["B"], OPT["lr"],
                                       OPT["b1"], OPT["b2"], OPT["eps"], OPT["wd"])
        rt.L.malus_gpt_set_fused_optimizer(self.g, int(fused))
        rt.L.malus_gpt_set_fused_forward(self.g, int(fused_forward))

    def close(self):
        self.rt.L.malus_gpt_free(self.g)
        self.rt.L.tape_reset()

    def param(self, i):
        return self.rt.numpy(self.rt.L.malus_gpt_param(self.g, i)).ravel()

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


def tokens(cfg, call_idx):
    n = cfg["B"] * cfg["T"]
    return O.rand_tokens(call_idx, n, cfg["V"]), O.rand_tokens(call_idx + n, n, cfg["V"])


def test_gpt_init_matches_oracle_bitexact(rt):
    g = GpuGpt(rt, C4)
    og = O.Gpt(**C4)
    try:
        for i in range(og.nparams):
            np.testing.assert_array_equal(g.param(i), og.param(i), err_msg=f"param {i}")
    finally:
        g.close()


def test_gpt_c4_loss_and_grads_vs_oracle(rt):
    g = GpuGpt(rt, C4)
    og = O.Gpt(**C4)
    O.set_threads(oracle_threads())
    x, y = tokens(C4, 1 << 20)
    try:
        loss = g.loss_and_grads(x, y)
        wloss = og.loss_and_grads(x, y)
        worst = max(normwise_err(g.grad(i), og.grad(i)) for i in range(og.nparams))
        print(f"loss rel {abs(loss - wloss) / abs(wloss):.2e}, worst normwise gradient error {worst:.2e}")
        assert abs(loss - wloss) <= 1e-5 * abs(wloss), (loss, wloss)
        assert worst <= 3e-5, f"worst normwise gradient error {worst:.2e}"
    finally:
        g.close()


def test_gpt_fused_optimizer_equals_op_by_op(rt):
    cfg = dict(V=65, T=16, C=32, H=4, L=2, B=4)
    x, y = tokens(cfg, 5000)
    a, b = GpuGpt(rt, cfg, fused=True), None
    try:
        la = [a.step(x, y, t) for t in (1, 2)]
        pa = [a.param(i) for i in range(8 * cfg["L"] + 4)]
    finally:
        a.close()
    b = GpuGpt(rt, cfg, fused=False)
    try:
        lb = [b.step(x, y, t) for t in (1, 2)]
        pb = [b.param(i) for i in range(8 * cfg["L"] + 4)]
    finally:
        b.close()
    assert la == lb
    for i, (u, v) in enumerate(zip(pa, pb)):
        np.testing.assert_array_equal(u, v, err_msg=f"param {i}")


@pytest.mark.parametrize("cfg", [dict(V=65, T=64, C=64, H=4, L=2, B=4),     # hs 16: GEMM + fused softmax
                                 dict(V=65, T=64, C=128, H=4, L=2, B=4),    # hs 32: fused scores kernel
                                 dict(V=65, T=256, C=128, H=2, L=1, B=2),   # hs 64, T 256: fused scores kernel
                                 dict(V=65, T=128, C=256, H=4, L=2, B=3),   # hs 64, T 128
                                 dict(V=65, T=64, C=384, H=6, L=1, B=16),   # C5 width: LN-scale VJP at 384 columns
                                 dict(V=65, T=20, C=384, H=6, L=1, B=3),    # 60 rows: a ragged last row block
                                 dict(V=65, T=16, C=512, H=8, L=1, B=6),    # 512 columns
                                 # the LN-scale VJP's column partials over 198 and 300 row chunks: combined in
                                 # two lane steps, singly (198) and in runs of four (300)
                                 dict(V=65, T=64, C=384, H=6, L=1, B=99),
                                 dict(V=65, T=64, C=384, H=6, L=1, B=150)],
                         ids=["t64hs16", "t64hs32", "t256hs64", "t128hs64", "c384", "c384ragged", "c512", "c384s198",
                              "c384s300"])
def test_gpt_fusions_equal_separate_ops(rt, cfg):
    """The forward fusions (attention scores + scale + mask + softmax in one
    kernel where the head size allows it, else scale + mask + softmax in one
    kernel; residual adds in GEMM epilogues; shape-only intermediates on the
    tape) and the VJP fusions (gradient accumulation inside the matmul /
    layernorm VJP kernels) give the same loss, gradients and updated
    parameters as the separate ops, bit for bit."""
    x, y = tokens(cfg, 6000)
    out = []
    for fa in (True, False):
        rt.L.malus_tape_set_fused_vjps(int(fa))
        g = GpuGpt(rt, cfg, fused_forward=fa)
        rt.L.malus_gpt_set_attention(g.g, 2)  # the row-register fused kernels where built (not flash)
        try:
            loss = g.loss_and_grads(x, y)
            grads = [g.grad(i) for i in range(8 * cfg["L"] + 4)]
            l2 = g.step(x, y, 1)
            params = [g.param(i) for i in range(8 * cfg["L"] + 4)]
        finally:
            g.close()
            rt.L.malus_tape_set_fused_vjps(1)
        out.append((loss, grads, l2, params))
    (la, ga, sa, pa), (lb, gb, sb, pb) = out
    assert la == lb and sa == sb
    for i in range(len(ga)):
        np.testing.assert_array_equal(ga[i], gb[i], err_msg=f"grad {i}")
        np.testing.assert_array_equal(pa[i], pb[i], err_msg=f"param {i}")


@pytest.mark.parametrize("cfg", [dict(V=65, T=256, C=128, H=2, L=2, B=2),
                                 dict(V=65, T=128, C=256, H=4, L=1, B=3)], ids=["t256hs64", "t128hs64"])
def test_fused_attention_unwritten_tiles(rt, cfg):
    """The fused attention forward leaves P's 32 x 32 tiles wholly above the
    diagonal unwritten.  With the pool's buffers of P's size poisoned with
    NaN, the fused VJP (which reads only the other tiles) and the composed
    VJPs (GEMMs over P after the runtime fills those tiles with zeros) must
    give the same gradients, bit for bit, and finite."""
    x, y = tokens(cfg, 7000)
    nbytes = cfg["B"] * cfg["H"] * cfg["T"] * cfg["T"]
    out = []
    for fv in (True, False):
        poison = [rt.tensor(np.full(nbytes, np.nan, np.float32)) for _ in range(2 * cfg["L"])]
        rt.free(*poison)
        rt.L.malus_tape_set_fused_vjps(int(fv))
        g = GpuGpt(rt, cfg, fused_forward=True)
        rt.L.malus_gpt_set_attention(g.g, 2)  # the row-register fused kernels
        try:
            loss = g.loss_and_grads(x, y)
            grads = [g.grad(i) for i in range(8 * cfg["L"] + 4)]
        finally:
            g.close()
            rt.L.malus_tape_set_fused_vjps(1)
        out.append((loss, grads))
    (la, ga), (lb, gb) = out
    assert np.isfinite(la) and la == lb
    for i in range(len(ga)):
        assert np.all(np.isfinite(ga[i])), f"grad {i}"
        np.testing.assert_array_equal(ga[i], gb[i], err_msg=f"grad {i}")


def test_gpt_c4_200_step_loss_trajectory(rt):
    g = GpuGpt(rt, C4)
    og = O.Gpt(**C4)
    O.set_threads(oracle_threads())
    try:
        worst = 0.0
        for t in range(1, 201):
            x, y = tokens(C4, 10_000_000 + 2 * 2048 * t)
            lg = g.step(x, y, t)
            lo = og.step(x, y, t)
            worst = max(worst, abs(lg - lo) / abs(lo))
            assert worst <= 1e-3, f"step {t}: {lg} vs {lo}"
        print(f"C4 200-step worst relative loss difference {worst:.2e}")
    finally:
        g.close()


def test_gpt_c5_one_step_vs_oracle(rt):
    g = GpuGpt(rt, C5)
    og = O.Gpt(**C5)
    O.set_threads(oracle_threads())
    x, y = tokens(C5, 1 << 24)
    try:
        loss = g.loss_and_grads(x, y)
        wloss = og.loss_and_grads(x, y)
        worst = max(normwise_err(g.grad(i), og.grad(i)) for i in range(og.nparams))
        print(f"loss rel {abs(loss - wloss) / abs(wloss):.2e}, worst normwise gradient error {worst:.2e}")
        assert abs(loss - wloss) <= 1e-5 * abs(wloss), (loss, wloss)
        assert worst <= 3e-5, f"worst normwise gradient error {worst:.2e}"
    finally:
        g.close()


# ------------------------------------------------------ C5 over many steps
def _c5_fixture(name):
    import json
    import pathlib

    fx = json.loads((pathlib.Path(__file__).parent / "golden" / name).read_text())
    assert fx["config"] == C5 and fx["optimizer"] == OPT
    return fx


def _c5_model(rt):
    rt.L.tape_reset()
    rt.L.malus_rng_set_counter(0)
    return rt.L.malus_gpt_create(C5["V"], C5["T"], C5["C"], C5["H"], C5["L"], C5["B"], OPT["lr"], OPT["b1"],
                                 OPT["b2"], OPT["eps"], OPT["wd"])


def _c5_corpus_losses(rt, steps, autocast):
    """C5 steps as the bench runs them (one capture, then replays) on the
    corpus batches of tests/golden/make_c5_trajectory.py."""
    from tests.golden.make_c5_trajectory import batch, checksum, corpus

    fx = _c5_fixture("c5_trajectory.json")
    data = corpus()
    I32P = C.POINTER(C.c_int32)
    g = _c5_model(rt)
    losses, gr = [], None
    try:
        with M.autocast(autocast):
            for t in range(1, steps + 1):
                x, y = batch(data, t)
                assert checksum(x, y) == fx["batch_checksums"][t - 1], f"step {t}: not the fixture's batch"
                if gr is None:
                    l0 = C.c_int64()
                    gr = rt.L.malus_gpt_graph_create(g, x.ctypes.data_as(I32P), y.ctypes.data_as(I32P), t, C.byref(l0))
                    assert gr, rt.last_error()
                    h = l0.value
                else:
                    h = rt.L.malus_gpt_graph_step(gr, x.ctypes.data_as(I32P), y.ctypes.data_as(I32P), t)
                    assert h, rt.last_error()
                losses.append(float(rt.numpy(h)[0]))
                rt.free(h)
    finally:
        if gr:
            rt.L.malus_gpt_graph_free(gr)
        rt.L.malus_gpt_free(g)
        rt.L.tape_reset()
    return np.array(losses), np.array(fx["losses"][:steps])


def test_gpt_c5_200_step_trajectory_vs_oracle_fixture(rt):
    """The north star's trajectory bar on the configuration's own data: 200
    replays of the captured C5 step, each drawing its i.i.d. ids on the
    device (the bench's path), every loss within 1e-3 relative of the CPU
    oracle's (tests/golden/c5_trajectory_iid.json)."""
    from tests.golden.make_c5_trajectory import N_TOK, checksum, iid_calls

    fx = _c5_fixture("c5_trajectory_iid.json")
    want = np.array(fx["losses"])
    assert len(want) == 200
    for t in (1, 200):  # the device draw is the fixture's batch
        hx, hy = (rt.L.malus_rand_tokens_device(c, N_TOK, C5["V"]) for c in iid_calls(t))
        assert checksum(rt.numpy(hx), rt.numpy(hy)) == fx["batch_checksums"][t - 1]
        rt.free(hx, hy)
    g = _c5_model(rt)
    got, gr = [], None
    try:
        for t in range(1, 201):
            cx, cy = iid_calls(t)
            if gr is None:
                l0 = C.c_int64()
                gr = rt.L.malus_gpt_graph_create_drawn(g, cx, cy, t, C.byref(l0))
                assert gr, rt.last_error()
                h = l0.value
            else:
                h = rt.L.malus_gpt_graph_step_drawn(gr, cx, cy, t)
                assert h, rt.last_error()
            got.append(float(rt.numpy(h)[0]))
            rt.free(h)
    finally:
        if gr:
            rt.L.malus_gpt_graph_free(gr)
        rt.L.malus_gpt_free(g)
        rt.L.tape_reset()
    got = np.array(got)
    rel = np.abs(got - want) / want
    print(f"C5 200 steps (i.i.d. ids): loss {got[0]:.5f} -> {got[-1]:.5f} (oracle {want[0]:.5f} -> {want[-1]:.5f}); "
          f"worst relative difference {rel.max():.2e} at step {int(rel.argmax()) + 1}")
    assert want[-1] < want[0]
    assert rel.max() <= 1e-3


def test_gpt_c5_learning_trajectory_vs_oracle_fixture(rt):
    """On the learnable corpus the loss falls from 4.26 to ~1.8 by step 45,
    through a transition (steps ~20-40) where runs whose sums differ in the
    last bit take measurably different paths (two f32 implementations part
    by up to ~1e-2 there and ~3e-2 once the run turns unstable near step 85
    at this learning rate).  So: every step within 1e-3 of the oracle up to
    step 20, the learned plateau (the mean loss over steps 41-80) within 1 %
    of the oracle's, and the corpus learned."""
    got, want = _c5_corpus_losses(rt, 80, False)
    rel = np.abs(got - want) / want
    plateau = abs(got[40:80].mean() - want[40:80].mean()) / want[40:80].mean()
    print(f"C5 corpus: steps 1-20 worst relative difference {rel[:20].max():.2e}; plateau (41-80) mean "
          f"{got[40:80].mean():.4f} vs oracle {want[40:80].mean():.4f} ({plateau:.2e})")
    assert rel[:20].max() <= 1e-3
    assert plateau <= 0.01
    assert got[49] < 0.5 * got[0] and want[49] < 0.5 * want[0]


def test_autocast_c5_convergence_parity(rt):
    # docs/adr/0037-bf16-autocast.md:12: bf16 autocast converges with the f32
    # run "within noise": every step up to 20 within 2 % of the f32 oracle,
    # the learned plateau (mean over steps 41-80) within 2 % of the oracle's,
    # and the corpus learned as in f32
    got, want = _c5_corpus_losses(rt, 80, True)
    rel = np.abs(got - want) / want
    plateau = abs(got[40:80].mean() - want[40:80].mean()) / want[40:80].mean()
    print(f"autocast C5 corpus: steps 1-20 worst relative difference {rel[:20].max():.2e}; plateau (41-80) mean "
          f"{got[40:80].mean():.4f} vs f32 oracle {want[40:80].mean():.4f} ({plateau:.2e})")
    assert rel[:20].max() <= 0.02
    assert plateau <= 0.02
    assert got[49] < 0.5 * got[0]
