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


def test_failed_graph_create_leaves_eager_steps_unchanged(rt):
    """A create that fails inside its capture (an allocation failure injected
    on the host) returns null with the error, releases what it holds and
    detaches from the model: later eager steps use their own AdamW bias
    corrections again, so they equal a model that never had a graph."""
    cfg = dict(V=65, T=64, C=128, H=4, L=2, B=4)
    n = cfg["B"] * cfg["T"]
    batches = [(O.rand_tokens(700 + 2 * k, n, cfg["V"]), O.rand_tokens(701 + 2 * k, n, cfg["V"])) for k in range(3)]
    I32 = lambda a: a.ctypes.data_as(I32P)  # noqa: E731
    stats = (C.c_int64 * 4)()

    def allocs():
        rt.L.malus_pool_stats(stats)
        return stats[0] + stats[1]

    # pool allocations of a whole create (its eager step, then the capture of the same body)
    g = make(rt, cfg)
    a0 = allocs()
    gr = rt.L.malus_gpt_graph_create(g, I32(batches[0][0]), I32(batches[0][1]), 1, None)
    assert gr, rt.last_error()
    per_create = allocs() - a0
    rt.L.malus_gpt_graph_free(gr)
    rt.L.malus_gpt_free(g)
    rt.L.tape_reset()

    # reference: three eager steps
    g = make(rt, cfg)
    want = []
    for k, (x, y) in enumerate(batches):
        hx, hy = rt.tensor(x), rt.tensor(y)
        hl = rt.L.malus_gpt_step(g, hx, hy, k + 1)
        want.append(rt.numpy(hl)[0])
        rt.free(hl, hx, hy)
    want_state = state(rt, g)
    rt.L.malus_gpt_free(g)
    rt.L.tape_reset()

    # step 1 inside a create whose capture fails three quarters of the way through
    g = make(rt, cfg)
    live = rt.L.malus_pool_live_bytes()
    rt.L.malus_set_abort_on_error(0)
    try:
        rt.L.malus_fail_alloc_after(per_create * 3 // 4)
        gr = rt.L.malus_gpt_graph_create(g, I32(batches[0][0]), I32(batches[0][1]), 1, None)
        rt.L.malus_fail_alloc_after(-1)
        assert not gr
        assert "injected allocation failure" in rt.last_error()
        rt.L.malus_clear_error()
    finally:
        rt.L.malus_fail_alloc_after(-1)
        rt.L.malus_set_abort_on_error(1)
    got = []
    for k, (x, y) in enumerate(batches[1:], start=2):
        hx, hy = rt.tensor(x), rt.tensor(y)
        hl = rt.L.malus_gpt_step(g, hx, hy, k)
        got.append(rt.numpy(hl)[0])
        rt.free(hl, hx, hy)
    got_state = state(rt, g)
    rt.L.malus_gpt_free(g)
    rt.L.tape_reset()
    np.testing.assert_array_equal(np.array(got), np.array(want[1:]))
    for i, (a, b) in enumerate(zip(got_state, want_state)):
        assert np.array_equal(a, b), f"state tensor {i} differs after a failed graph create"
    # what the graph held is back in the pool (the handles of the step that
    # was cut short, at most a few of this config's sub-megabyte tensors, are
    # not reachable to free)
    assert rt.L.malus_pool_live_bytes() <= live + (8 << 20)


C5 = dict(V=65, T=256, C=384, H=6, L=6, B=64)


@pytest.mark.parametrize("autocast,attention", [(False, 2), (False, 0), (True, 0)],
                         ids=["f32_rows_attention", "f32_auto_flash_attention", "autocast_flash"])
def test_c5_graph_replays_equal_eager_steps(rt, autocast, attention):
    """The headline workload as the bench runs it: C5 (examples/nanogpt_modular.ml
    step, lines 167-189) captured once with its token draw and replayed.  At
    B*T = 16,384 tokens the weight-gradient GEMMs split K (partials summed by
    the split reduction in pool memory the capture reserves), the q/k/v
    projections run grouped, and the attention is the row-register kernel
    pair (its tiles above the diagonal left unwritten) or flash attention
    (the automatic choice at C5, in f32 with split products and under
    autocast).  The replayed steps draw their ids on the
    device (call indices past 2^32, so both key words move); eager steps get
    the oracle's draw of the same calls uploaded.  Replays equal eager steps
    bit for bit (losses, parameters, both moments); in f32 the first two
    losses also match the oracle's steps at 1e-5."""
    steps = 4
    n = C5["B"] * C5["T"]
    calls = [((1 << 32) - n // 2 + 2 * n * k, (1 << 32) - n // 2 + 2 * n * k + n) for k in range(steps)]
    batches = [(O.rand_tokens(cx, n, C5["V"]), O.rand_tokens(cy, n, C5["V"])) for cx, cy in calls]
    with M.autocast(autocast):
        g = make(rt, C5)
        rt.L.malus_gpt_set_attention(g, attention)
        eager = []
        for k, (x, y) in enumerate(batches):
            hx, hy = rt.tensor(x), rt.tensor(y)
            hl = rt.L.malus_gpt_step(g, hx, hy, k + 1)
            eager.append(rt.numpy(hl)[0])
            rt.free(hl, hx, hy)
        eager_state = state(rt, g)
        rt.L.malus_gpt_free(g)
        rt.L.tape_reset()

        g = make(rt, C5)
        rt.L.malus_gpt_set_attention(g, attention)
        l0 = C.c_int64()
        gr = rt.L.malus_gpt_graph_create_drawn(g, calls[0][0], calls[0][1], 1, C.byref(l0))
        assert gr, rt.last_error()
        graph = [rt.numpy(l0.value)[0]]
        rt.free(l0.value)
        for k in range(1, steps):
            hl = rt.L.malus_gpt_graph_step_drawn(gr, calls[k][0], calls[k][1], k + 1)
            assert hl, rt.last_error()
            graph.append(rt.numpy(hl)[0])
            rt.free(hl)
        graph_state = state(rt, g)
        rt.L.malus_gpt_graph_free(gr)
        rt.L.malus_gpt_free(g)
        rt.L.tape_reset()
    print(f"C5 {'autocast' if autocast else 'f32'} attention {attention} losses: graph {graph} eager {eager}")
    np.testing.assert_array_equal(np.array(graph), np.array(eager))
    for i, (a, b) in enumerate(zip(graph_state, eager_state)):
        assert np.array_equal(a, b), f"state tensor {i} differs between the graph and the eager steps"
    if not autocast:
        og = O.Gpt(**C5)
        O.set_threads(16)
        for k in range(2):
            want = og.step(*batches[k], k + 1)
            assert abs(graph[k] - want) <= 1e-5 * want, (k + 1, graph[k], want)


def test_graph_kinds_refuse_the_other_step(rt):
    cfg = dict(V=33, T=16, C=32, H=4, L=1, B=2)
    n = cfg["B"] * cfg["T"]
    x = O.rand_tokens(5, n, cfg["V"])
    g = make(rt, cfg)
    gr = rt.L.malus_gpt_graph_create_drawn(g, 10, 10 + n, 1, None)
    assert gr, rt.last_error()
    rt.L.malus_set_abort_on_error(0)
    try:
        assert rt.L.malus_gpt_graph_step(gr, x.ctypes.data_as(I32P), x.ctypes.data_as(I32P), 2) == 0
        assert "draws its ids" in rt.last_error()
        rt.L.malus_clear_error()
        assert rt.L.malus_gpt_graph_create_drawn(g, 1, 2, 2, None) is None
        assert "already has a graph" in rt.last_error()
        rt.L.malus_clear_error()
    finally:
        rt.L.malus_set_abort_on_error(1)
    rt.L.malus_gpt_graph_free(gr)
    rt.L.malus_gpt_free(g)
    rt.L.tape_reset()
