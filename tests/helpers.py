"""Comparison helpers shared by the parity tests.

Tolerance rules (stated once, used by every test):
  * integer / index / permutation / +-*/ work: bit-exact;
  * transcendental elementwise ops: <= 2 ulp of the oracle (glibc libm vs
    the device math library, each ~1 ulp);
  * reductions, softmax, layernorm, matmul: normwise relative error
    max|got - want| <= rtol * max|want| with rtol = 1e-5 — summation order
    differs (tree vs sequential), so elementwise relative error is not
    meaningful near zero;
  * reductions over long axes (assert_reduction): within 1e-5 normwise of
    the float64 exact result, or no farther from it than the sequential f32
    reference result is (that result alone drifts ~1e-5 at n ~ 70k).
"""
import numpy as np
import json as _json
import pathlib as _pathlib

# Known answers from the reference's tests and README (see the fixture's
# "source" fields).
KATS = _json.loads((_pathlib.Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def ulp_dist(a, b):
    a = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    # map sign-magnitude to a monotonic integer line
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return np.abs(a - b)


def assert_bitexact(got, want, what=""):
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    if got.dtype == np.float32:
        bad = (got.view(np.int32) != want.astype(np.float32).view(np.int32)) & ~(np.isnan(got) & np.isnan(want))
    else:
        bad = got != want
    n = int(np.count_nonzero(bad))
    if n:
        i = int(np.flatnonzero(bad)[0])
        raise AssertionError(f"{what}: {n} of {got.size} elements differ; first at {i}: {got.ravel()[i]!r} vs {want.ravel()[i]!r}")


def assert_ulp(got, want, max_ulp=2, what=""):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    d = ulp_dist(got, want)
    d = np.where(np.isnan(got) & np.isnan(want), 0, d)
    worst = int(d.max()) if d.size else 0
    if worst > max_ulp:
        i = int(np.argmax(d))
        raise AssertionError(f"{what}: {worst} ulp > {max_ulp} at {i}: {got.ravel()[i]!r} vs {want.ravel()[i]!r}")


def normwise_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = max(float(np.max(np.abs(want))) if want.size else 0.0, 1e-30)
    return float(np.max(np.abs(got - want))) / scale if want.size else 0.0


def assert_reduction(got, oracle_out, exact, rtol=1e-5, what=""):
    """Reductions over long axes: the sequential f32 oracle itself drifts
    ~sqrt(n)*eps from the exact sum (n = 70k: ~1e-5), so the GPU result must
    be within rtol normwise of the float64 exact value, or no farther from it
    than the reference's own sequential-f32 result is."""
    got = np.asarray(got, np.float64)
    exact = np.asarray(exact, np.float64)
    assert np.all(np.isfinite(got)), f"{what}: non-finite values in the GPU result"
    scale = max(float(np.max(np.abs(exact))), 1e-30)
    ref_err = float(np.max(np.abs(np.asarray(oracle_out, np.float64) - exact)))
    err = float(np.max(np.abs(got - exact)))
    assert err <= max(rtol * scale, ref_err), (
        f"{what}: GPU error vs exact {err / scale:.3e} exceeds both {rtol:.0e} and the reference's own {ref_err / scale:.3e}")


def assert_normwise(got, want, rtol=1e-5, what=""):
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    assert np.all(np.isfinite(got)), f"{what}: non-finite values in the GPU result"
    e = normwise_err(got, want)
    assert e <= rtol, f"{what}: normwise relative error {e:.3e} > {rtol:.0e}"
