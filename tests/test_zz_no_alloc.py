"""GPU test of malus_std_reduce_noalloc, the allocation-free variant of
malus_std_reduce_fwd: for every op and each reduction path (long rows split
across workgroups, one wave per row, column reductions with split partials),
two calls in a row, the second with a smaller input, each equal bit for bit
to malus_std_reduce_fwd on the same input (same kernels, same plan) and
within the reduction bar of the oracle; a reduction needing more than the
fixed scratch array is rejected with an error."""
import numpy as np
import pytest

import malus_amd as M
from oracle import oracle as O
from tests.helpers import assert_bitexact, assert_reduction

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(2026)

# (first call: shape, axis), (second call, smaller: shape, axis)
CASES = [
    (((64, 50000), 1), ((8, 20000), 1)),        # long rows: split across workgroups, partials in scratch
    (((65536, 64), 0), ((9000, 48), 0)),        # column reduction with split partials
    (((3, 4000, 96), 1), ((2, 1000, 8), 1)),    # outer > 1, split partials
    (((500, 1024), 1), ((7, 33), -1)),          # one wave per row (no scratch)
]


def out_shape(shape, axis):
    ax = axis % len(shape)
    return tuple(d for i, d in enumerate(shape) if i != ax) or (1,)


def noalloc(rt, op, hx, shape, axis):
    osh = out_shape(shape, axis)
    hout = rt.L.tensor_alloc_gpu(M.F32, M.sizes(osh), len(osh), None)
    rc = rt.L.malus_std_reduce_noalloc(op, rt.L.malus_tensor_device_ptr(hx), M.sizes(shape), len(shape), axis,
                                       rt.L.malus_tensor_device_ptr(hout))
    assert rc == 0, rt.last_error()
    rt.L.gpu_barrier()  # the result is on the library's stream
    out = rt.numpy(hout)
    rt.free(hout)
    return out


@pytest.mark.parametrize("op", [M.R_SUM, M.R_MEAN, M.R_MAX, M.R_VAR])
@pytest.mark.parametrize("first,second", CASES, ids=[f"{c[0][0]}ax{c[0][1]}" for c in CASES])
def test_noalloc_reduce_matches_reduce_fwd_twice(rt, op, first, second):
    for shape, axis in (first, second):
        x = RNG.uniform(-2, 2, shape).astype(np.float32)
        hx = rt.tensor(x)
        got = noalloc(rt, op, hx, shape, axis)
        want_h = rt.L.malus_std_reduce_fwd(op, hx, axis, 0)
        want = rt.numpy(want_h)
        rt.free(want_h)
        assert_bitexact(got, want.reshape(got.shape), f"noalloc vs reduce_fwd op {op} {shape} axis {axis}")
        if x.size <= 1 << 22:
            ref = O.reduce_axis(op, x, axis).reshape(got.shape)
            if op == M.R_MAX:
                assert_bitexact(got, ref, "max vs oracle")
            else:
                x64 = x.astype(np.float64)
                exact = {M.R_SUM: x64.sum, M.R_MEAN: x64.mean, M.R_VAR: x64.var}[op](axis=axis).reshape(got.shape)
                assert_reduction(got, ref, exact, 1e-5, f"noalloc op {op} vs oracle")
        rt.free(hx)


def test_noalloc_rejects_reductions_past_the_scratch_array(rt):
    shape = (2, (1 << 20) + 64)  # the variance's mean alone needs more than 4 MiB
    hx = rt.tensor(np.ones(shape, np.float32))
    hout = rt.L.tensor_alloc_gpu(M.F32, M.sizes((shape[1],)), 1, None)
    rt.L.malus_set_abort_on_error(0)
    try:
        rc = rt.L.malus_std_reduce_noalloc(M.R_VAR, rt.L.malus_tensor_device_ptr(hx), M.sizes(shape), 2, 0,
                                           rt.L.malus_tensor_device_ptr(hout))
        assert rc == -1
        assert "more than the 4194304-byte array" in rt.last_error()
        rt.L.malus_clear_error()
        rc = rt.L.malus_std_reduce_noalloc(7, rt.L.malus_tensor_device_ptr(hx), M.sizes(shape), 2, 0,
                                           rt.L.malus_tensor_device_ptr(hout))
        assert rc == -1 and "bad reduction op" in rt.last_error()
        rt.L.malus_clear_error()
    finally:
        rt.L.malus_set_abort_on_error(1)
    # the same reduction through the allocating entry point still works
    h = rt.L.malus_std_reduce_fwd(M.R_VAR, hx, 0, 0)
    assert np.all(rt.numpy(h) == 0.0)
    rt.free(h, hx, hout)


@pytest.mark.parametrize("shape,axis", [((65536, 64), 0), ((3, 4000, 96), 1)])
def test_noalloc_variance_with_unaligned_output(rt, shape, axis):
    # x 16-byte aligned, out 4 bytes past an aligned address: the variance's
    # mean pass plans with x and its own aligned mean, the second pass with
    # x, the mean and out, so the two passes take different column plans
    x = RNG.uniform(-2, 2, shape).astype(np.float32)
    hx = rt.tensor(x)
    osh = out_shape(shape, axis)
    n = int(np.prod(osh))
    hout = rt.L.tensor_alloc_gpu(M.F32, M.sizes((n + 1,)), 1, None)
    rc = rt.L.malus_std_reduce_noalloc(M.R_VAR, rt.L.malus_tensor_device_ptr(hx), M.sizes(shape), len(shape), axis,
                                       rt.L.malus_tensor_device_ptr(hout) + 4)
    assert rc == 0, rt.last_error()
    rt.L.gpu_barrier()
    got = rt.numpy(hout).ravel()[1:]
    want_h = rt.L.malus_std_reduce_fwd(M.R_VAR, hx, axis, 0)
    want = rt.numpy(want_h).ravel()
    rt.free(want_h, hout, hx)
    exact = x.astype(np.float64).var(axis=axis).ravel()
    assert_reduction(got, O.reduce_axis(M.R_VAR, x, axis).ravel(), exact, 1e-5, "unaligned-out variance vs oracle")
    assert_reduction(want, O.reduce_axis(M.R_VAR, x, axis).ravel(), exact, 1e-5, "reduce_fwd variance vs oracle")
