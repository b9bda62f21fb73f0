"""The training step as a HIP graph (malus_gpt_graph_*) against the eager
step (malus_gpt_step): the same losses and the same parameters and moments,
bit for bit, over several replays.  Between replays the test does eager
work of its own: it allocates and fills tensors of the step's sizes and
keeps them alive across a replay (the graph's buffers are reserved, so they
must come back unchanged), reads the loss, and runs unrelated ops."""
import ctypes as C

import numpy as np
import pytest

import malus_amd as M
from oracle import oracle as O
from tests.helpers import assert_normwise

pytestmark = pytest.mark.gpu

OPT = dict(lr=1e-3, b1=0.9, b2=0.99, eps=1e-8, wd=0.1)
I32P = C.POINTER(C.c_int32)


def make(rt, cfg):
    rt.L.tape_reset()
    rt.L.malus_rng_set_counter(0)
    return rt.L.malus_gpt_create(cfg["V"], cfg["T"], cfg["C"], cfg["H"], cfg["L"], cfg["B"], OPT["lr"], OPT["b1"],
                                 OPT["b2"], OPT["eps"], OPT["wd"])


def state(rt, g):
    out = []
    for i in range(rt.L.malus_gpt_nparams(g)):
        out.append(rt.numpy(rt.L.malus_gpt_param(g, i)))
        out.append(rt.numpy(rt.L.malus_gpt_moment(g, i, 0)))
        out.append(rt.numpy(rt.L.malus_gpt_moment(g, i, 1)))
    return out


@pytest.mark.parametrize("cfg", [dict(V=65, T=64, C=128, H=4, L=2, B=4),     # fused attention (T=64, hs=32)
                                 dict(V=33, T=16, C=32, H=4, L=2, B=3)],     # the composed attention path
                         ids=["fused_attention", "composed_attention"])
def test_graph_replays_equal_eager_steps(rt, cfg):
    n = cfg["B"] * cfg["T"]
    steps = 6
    batches = [(O.rand_tokens(500 + 2 * k, n, cfg["V"]), O.rand_tokens(501 + 2 * k, n, cfg["V"])) for k in range(steps)]

    # eager: malus_gpt_step with each step's token upload
    g = make(rt, cfg)
    eager_losses = []
    for k, (x, y) in enumerate(batches):
        hx, hy = rt.tensor(x), rt.tensor(y)
        hl = rt.L.malus_gpt_step(g, hx, hy, k + 1)
        eager_losses.append(rt.numpy(hl)[0])
        rt.free(hl, hx, hy)
    eager_state = state(rt, g)
    rt.L.malus_gpt_free(g)
    rt.L.tape_reset()

    # captured: step 1 eager inside create, steps 2.. as replays
    g = make(rt, cfg)
    x, y = batches[0]
    l0 = C.c_int64()
    gr = rt.L.malus_gpt_graph_create(g, x.ctypes.data_as(I32P), y.ctypes.data_as(I32P), 1, C.byref(l0))
    assert gr, rt.last_error()
    assert rt.L.malus_gpt_graph_nodes(gr) > 20
    graph_losses = [rt.numpy(l0.value)[0]]
    rt.free(l0.value)
    rng = np.random.default_rng(9)
    for k in range(1, steps):
        # eager work between replays: tensors of the step's sizes, alive across the replay
        keep = [rt.tensor(np.full(s, 7.25, np.float32)) for s in [(n, cfg["C"]), (n, 4 * cfg["C"]), (n, cfg["V"])]]
        av = rng.standard_normal((64, 64)).astype(np.float32)
        a = rt.tensor(av)
        prod = rt.L.tensor_matmul(a, a)
        x, y = batches[k]
        hl = rt.L.malus_gpt_graph_step(gr, x.ctypes.data_as(I32P), y.ctypes.data_as(I32P), k + 1)
        assert hl, rt.last_error()
        graph_losses.append(rt.numpy(hl)[0])
        for h in keep:
            assert np.all(rt.numpy(h) == 7.25), "a replay wrote into memory it does not own"
        assert_normwise(rt.numpy(prod), O.matmul(av, av), 1e-5, "eager matmul between replays")
        rt.free(hl, a, prod, *keep)
    graph_state = state(rt, g)
    rt.L.malus_gpt_graph_free(gr)
    rt.L.malus_gpt_free(g)
    rt.L.tape_reset()

    np.testing.assert_array_equal(np.array(graph_losses), np.array(eager_losses))
    for i, (a, b) in enumerate(zip(graph_state, eager_state)):
        assert np.array_equal(a, b), f"state tensor {i} differs between the graph and the eager steps"
    assert eager_losses[-1] < eager_losses[0]
