"""Flash attention (malus_std_flash_attn_fwd / _bwd, the model's attention
mode 1) against the composed attention of examples/nanogpt_modular.ml:57-62
as the oracle restates it: S = q @ k^T * scale + mask (tensor_causal_mask's
-1e9 above the diagonal), P = softmax(S, 2), out = P @ v; and the VJPs of
that chain: dP = dout @ v^T, dS = softmax_bwd(P, dP) * scale, dq = dS @ k,
dk = dS^T @ q, dv = P^T @ dout.

Tolerance: normwise 1e-5 (the online softmax rescales partial sums, and the
backward uses rowsum(dout * out) for rowsum(dP * P): equal in exact
arithmetic, different f32 rounding).  The row log-sum-exp is checked
against float64 within 2e-6 relative."""
import ctypes as C
import os

import numpy as np
import pytest

import malus_amd as M
from oracle import oracle as O
from tests.helpers import assert_normwise, normwise_err

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(29)
OPT = dict(lr=1e-3, b1=0.9, b2=0.99, eps=1e-8, wd=0.1)


def rand(*shape, lo=-1.0, hi=1.0):
    return RNG.uniform(lo, hi, size=shape).astype(np.float32)


def run(rt, h):
    out = rt.numpy(h)
    rt.free(h)
    return out


def composed(q, k, v, sc, causal):
    t = q.shape[1]
    s = O.matmul(q, np.ascontiguousarray(k.transpose(0, 2, 1)))
    s = O.broadcast(O.MUL, s, np.array([[sc]], np.float32))
    if causal:
        s = O.broadcast(O.ADD, s, O.causal_mask(t))
    p = O.softmax(s, 2)
    return s, p, O.matmul(p, v)


def composed_bwd(q, k, v, p, d, sc):
    dp = O.matmul(d, np.ascontiguousarray(v.transpose(0, 2, 1)))
    ds = O.broadcast(O.MUL, O.softmax_bwd(p, dp, 2), np.array([[sc]], np.float32))
    dq = O.matmul(ds, k)
    dk = O.matmul(np.ascontiguousarray(ds.transpose(0, 2, 1)), q)
    dv = O.matmul(np.ascontiguousarray(p.transpose(0, 2, 1)), d)
    return dq, dk, dv


SHAPES = [(6, 64, 32, 1), (6, 64, 32, 0), (5, 128, 64, 1), (4, 256, 64, 1), (4, 256, 64, 0), (3, 96, 64, 1),
          (2, 512, 64, 1), (1, 1024, 32, 1), (2, 32, 64, 1),
          (2, 1024, 64, 1), (1, 1024, 64, 0)]  # T >= 1024: the dQ pass runs four query tiles per workgroup


@pytest.mark.parametrize("bh,t,hs,causal", SHAPES, ids=[f"bh{a}t{b}hs{c}{'c' if d else 'n'}" for a, b, c, d in SHAPES])
def test_flash_fwd_bwd_vs_composed(rt, bh, t, hs, causal):
    O.set_threads(min(16, os.cpu_count() or 1))
    q, k, v = (rand(bh, t, hs, lo=-2, hi=2) for _ in range(3))
    d = rand(bh, t, hs)
    sc = float(np.float32(1.0 / np.sqrt(hs)))
    hq, hk, hv, hd = (rt.tensor(a) for a in (q, k, v, d))
    hsc = rt.tensor(np.array([[sc]], np.float32))
    hl = C.c_int64()
    ho = rt.L.malus_std_flash_attn_fwd(hq, hk, hv, hsc, causal, C.byref(hl))
    assert ho, rt.last_error()
    out, lse = rt.numpy(ho), rt.numpy(hl.value)
    s, p, want = composed(q, k, v, sc, causal)
    assert_normwise(out, want, 1e-5, f"flash out t={t} hs={hs} causal={causal}")
    s64 = s.astype(np.float64)
    mx = s64.max(2, keepdims=True)
    lse64 = (mx + np.log(np.exp(s64 - mx).sum(2, keepdims=True)))[..., 0]
    np.testing.assert_allclose(lse, lse64, rtol=2e-6, atol=2e-6)

    dq, dk, dv = C.c_int64(), C.c_int64(), C.c_int64()
    assert rt.L.malus_std_flash_attn_bwd(hd, hq, hk, hv, ho, hl.value, hsc, causal, 0, 0, 0, C.byref(dq), C.byref(dk),
                                         C.byref(dv)) == 0, rt.last_error()
    wq, wk, wv = composed_bwd(q, k, v, p, d, sc)
    assert_normwise(run(rt, dq.value), wq, 1e-5, "flash dq")
    assert_normwise(run(rt, dk.value), wk, 1e-5, "flash dk")
    assert_normwise(run(rt, dv.value), wv, 1e-5, "flash dv")
    rt.free(hq, hk, hv, hd, hsc, ho, hl.value)


def test_flash_bwd_addends(rt):
    bh, t, hs = 3, 128, 64
    q, k, v, d, aq, ak, av = (rand(bh, t, hs) for _ in range(7))
    sc = float(np.float32(0.125))
    hs_ = [rt.tensor(a) for a in (q, k, v, d, aq, ak, av)]
    hq, hk, hv, hd, haq, hak, hav = hs_
    hsc = rt.tensor(np.array([[sc]], np.float32))
    hl = C.c_int64()
    ho = rt.L.malus_std_flash_attn_fwd(hq, hk, hv, hsc, 1, C.byref(hl))
    outs = []
    for adds in ((0, 0, 0), (haq, hak, hav)):
        dq, dk, dv = C.c_int64(), C.c_int64(), C.c_int64()
        assert rt.L.malus_std_flash_attn_bwd(hd, hq, hk, hv, ho, hl.value, hsc, 1, *adds, C.byref(dq), C.byref(dk),
                                             C.byref(dv)) == 0
        outs.append([run(rt, h.value) for h in (dq, dk, dv)])
    for base, added, a in zip(outs[0], outs[1], (aq, ak, av)):
        np.testing.assert_array_equal(added, a + base)  # the addend is one f32 add of the same product
    rt.free(*hs_, hsc, ho, hl.value)


def test_flash_rejects_unsupported_shapes(rt):
    hq = rt.tensor(rand(2, 48, 64))  # t not a multiple of 32
    hsc = rt.tensor(np.array([[0.125]], np.float32))
    rt.L.malus_set_abort_on_error(0)
    try:
        assert rt.L.malus_std_flash_attn_fwd(hq, hq, hq, hsc, 1, None) == 0
        assert "multiple of 32" in rt.last_error()
        rt.L.malus_clear_error()
    finally:
        rt.L.malus_set_abort_on_error(1)
    rt.free(hq, hsc)


def test_flash_autocast_rounds_operands(rt):
    bh, t, hs = 4, 256, 64
    q, k, v = (rand(bh, t, hs, lo=-2, hi=2) for _ in range(3))
    sc = float(np.float32(0.125))
    hq, hk, hv = (rt.tensor(a) for a in (q, k, v))
    hsc = rt.tensor(np.array([[sc]], np.float32))
    with M.autocast():
        got = run(rt, rt.L.malus_std_flash_attn_fwd(hq, hk, hv, hsc, 1, None))
    f32 = run(rt, rt.L.malus_std_flash_attn_fwd(hq, hk, hv, hsc, 1, None))
    _, _, want = composed(q, k, v, sc, 1)
    e = normwise_err(got, want)
    print(f"autocast flash forward: normwise error {e:.2e} vs the f32 composed attention")
    assert 1e-4 < e < 2e-2  # bf16 operands (2^-9 relative each), f32 softmax and accumulation
    assert_normwise(f32, want, 1e-5, "f32 after the scope")
    rt.free(hq, hk, hv, hsc)


# ------------------------------------------------------------------- model
C4 = dict(V=65, T=64, C=128, H=4, L=4, B=32)
C5 = dict(V=65, T=256, C=384, H=6, L=6, B=64)


def gpt(rt, cfg, mode):
    rt.L.tape_reset()
    rt.L.malus_rng_set_counter(0)
    g = rt.L.malus_gpt_create(cfg["V"], cfg["T"], cfg["C"], cfg["H"], cfg["L"], cfg["B"], OPT["lr"], OPT["b1"],
                              OPT["b2"], OPT["eps"], OPT["wd"])
    assert rt.L.malus_gpt_set_attention(g, mode) == 0
    return g


def loss_and_grads(rt, g, cfg, x, y):
    hx, hy = rt.tensor(x), rt.tensor(y)
    rt.L.malus_gpt_zero_grad(g)
    hl = rt.L.malus_gpt_forward_loss(g, hx, hy)
    rt.L.backward(hl)
    loss = rt.numpy(hl)[0]
    grads = []
    for i in range(8 * cfg["L"] + 4):
        gh = rt.L.tape_get_grad(rt.L.malus_gpt_param(g, i))
        grads.append(rt.numpy(gh).ravel())
        rt.free(gh)
    rt.free(hx, hy, hl)
    return loss, grads


@pytest.mark.parametrize("cfg", [C4, C5, dict(V=65, T=512, C=128, H=2, L=2, B=2)], ids=["c4", "c5", "t512"])
def test_gpt_flash_attention_vs_oracle(rt, cfg):
    n = cfg["B"] * cfg["T"]
    x, y = O.rand_tokens(7 << 20, n, cfg["V"]), O.rand_tokens(9 << 20, n, cfg["V"])
    og = O.Gpt(**cfg)
    O.set_threads(min(16, os.cpu_count() or 1))
    wloss = og.loss_and_grads(x, y)
    g = gpt(rt, cfg, 1)
    try:
        loss, grads = loss_and_grads(rt, g, cfg, x, y)
    finally:
        rt.L.malus_gpt_free(g)
        rt.L.tape_reset()
    worst = max(normwise_err(grads[i], og.grad(i)) for i in range(og.nparams))
    print(f"flash {cfg}: loss {loss:.7f} oracle {wloss:.7f}, worst gradient error {worst:.2e}")
    assert abs(loss - wloss) <= 1e-5 * abs(wloss)
    assert worst <= 3e-5  # the model tests' gradient bar (measured 1.7e-6 .. 5.2e-6)


def test_gpt_flash_steps_deterministic_and_graph_equal(rt):
    """Two flash-attention models from the same seed give bit-identical
    steps (no atomics in the backward), eager and captured."""
    cfg = dict(V=65, T=128, C=128, H=2, L=2, B=4)
    n = cfg["B"] * cfg["T"]
    batches = [(O.rand_tokens(300 + 2 * s, n, cfg["V"]), O.rand_tokens(301 + 2 * s, n, cfg["V"])) for s in range(4)]
    runs = []
    for _ in range(2):
        g = gpt(rt, cfg, 1)
        losses = []
        for t, (x, y) in enumerate(batches, 1):
            hx, hy = rt.tensor(x), rt.tensor(y)
            hl = rt.L.malus_gpt_step(g, hx, hy, t)
            losses.append(rt.numpy(hl)[0])
            rt.free(hl, hx, hy)
        runs.append((losses, [rt.numpy(rt.L.malus_gpt_param(g, i)) for i in range(8 * cfg["L"] + 4)]))
        rt.L.malus_gpt_free(g)
        rt.L.tape_reset()
    assert runs[0][0] == runs[1][0]
    for a, b in zip(runs[0][1], runs[1][1]):
        np.testing.assert_array_equal(a, b)
    # captured: step 1 inside create, then replays
    I32P = C.POINTER(C.c_int32)
    g = gpt(rt, cfg, 1)
    l0 = C.c_int64()
    x, y = batches[0]
    gr = rt.L.malus_gpt_graph_create(g, x.ctypes.data_as(I32P), y.ctypes.data_as(I32P), 1, C.byref(l0))
    assert gr, rt.last_error()
    losses = [rt.numpy(l0.value)[0]]
    rt.free(l0.value)
    for t, (x, y) in enumerate(batches[1:], 2):
        hl = rt.L.malus_gpt_graph_step(gr, x.ctypes.data_as(I32P), y.ctypes.data_as(I32P), t)
        losses.append(rt.numpy(hl)[0])
        rt.free(hl)
    params = [rt.numpy(rt.L.malus_gpt_param(g, i)) for i in range(8 * cfg["L"] + 4)]
    rt.L.malus_gpt_graph_free(gr)
    rt.L.malus_gpt_free(g)
    rt.L.tape_reset()
    assert losses == runs[0][0]
    for a, b in zip(params, runs[0][1]):
        np.testing.assert_array_equal(a, b)
