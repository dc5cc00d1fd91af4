"""The DispatchTable forward kernels on the GPU (backend/dispatch.rs:51-93):
elementwise over the 21 ElementwiseKinds and reduction over the 6
ReductionKinds, full and per axis, against the oracle's restatement of the CPU
backend (backend/cpu/scalar.rs)."""
import numpy as np
import pytest

from numrs_amd import _lib as L
from oracle import oracle as O
from tests.conftest import assert_bits, assert_close

pytestmark = pytest.mark.gpu

EXACT = [L.EW_ADD, L.EW_MUL, L.EW_SUB, L.EW_DIV, L.EW_SQRT, L.EW_ABS, L.EW_NEG, L.EW_RELU,
         L.EW_LEAKY_RELU]
LIBM = [L.EW_POW, L.EW_SIN, L.EW_COS, L.EW_TAN, L.EW_ASIN, L.EW_ACOS, L.EW_ATAN, L.EW_EXP,
        L.EW_LOG, L.EW_SIGMOID, L.EW_TANH, L.EW_SOFTPLUS]
SPECIAL = np.array([0.0, -0.0, 1.5, -2.25, np.inf, -np.inf, np.nan, 1e-40, 3e38, -7.0],
                   np.float32)


def _inputs(kind, n, rng):
    a = rng.uniform(-3, 3, n).astype(np.float32)
    if kind in (L.EW_ASIN, L.EW_ACOS):
        a = rng.uniform(-1, 1, n).astype(np.float32)
    if kind in (L.EW_LOG, L.EW_POW, L.EW_SQRT):
        a = np.abs(a) + np.float32(0.01)
    b = rng.uniform(-2, 2, n).astype(np.float32)
    return a, b


@pytest.mark.parametrize("kind", EXACT + LIBM)
@pytest.mark.parametrize("n,off", [(100003, 0), (4099, 1)])
def test_elementwise(hip_ctx, kind, n, off):
    rng = np.random.default_rng(kind + 100)
    a, b = _inputs(kind, n, rng)
    if off == 0:  # special values through the aligned float4 path
        a[:SPECIAL.size], b[:SPECIAL.size] = SPECIAL, SPECIAL[::-1]
    c = hip_ctx
    ab = c.to_device(np.concatenate([np.zeros(off), a]).astype(np.float32))
    bb = c.to_device(np.concatenate([np.zeros(off), b]).astype(np.float32))
    ob = c.empty((n + off,))
    av, bv, ov = ab.view(off, (n,)), bb.view(off, (n,)), ob.view(off, (n,))
    c.elementwise(kind, av, bv, ov)
    want = O.elementwise(kind, a, b)
    got = ov.numpy()
    if kind in EXACT:
        assert_bits(got, want, f"kind {kind}")
    else:
        assert np.array_equal(np.isnan(got), np.isnan(want)), f"kind {kind} NaN pattern"
        fin = np.isfinite(want)
        assert np.array_equal(got[~fin & ~np.isnan(want)], want[~fin & ~np.isnan(want)])
        assert_close(got[fin], want[fin], abs_tol=1e-6, rel_tol=4e-6, what=f"kind {kind}")


KINDS = [L.RED_SUM, L.RED_MAX, L.RED_MIN, L.RED_MEAN, L.RED_ARGMAX, L.RED_VARIANCE]


@pytest.mark.parametrize("shape", [(7,), (33, 65), (4, 5, 6), (4096, 257), (3, 1000, 4)])
@pytest.mark.parametrize("kind", KINDS)
def test_reduction(hip_ctx, shape, kind):
    rng = np.random.default_rng(len(shape) * 10 + kind)
    x = rng.standard_normal(shape).astype(np.float32)
    c = hip_ctx
    xd = c.to_device(x)
    for axis in [None] + list(range(len(shape))):
        want = O.reduction(kind, x, axis)
        out = c.empty(want.shape)
        c.reduction(kind, xd, axis, out)
        got = out.numpy()
        n = x.size if axis is None else shape[axis]
        if kind in (L.RED_MAX, L.RED_MIN, L.RED_ARGMAX):
            assert_bits(got, want, f"kind {kind} axis {axis}")
        else:
            tol = 1e-5 + 4e-7 * n * (1.0 if kind != L.RED_MEAN else 1.0 / n)
            assert_close(got, want, abs_tol=tol, rel_tol=1e-4, what=f"kind {kind} axis {axis}")


def test_reduction_nan_rules(hip_ctx):
    nan = np.nan
    c = hip_ctx
    cases = [
        (L.RED_MAX, np.array([nan, 1, 3, nan], np.float32), None),
        (L.RED_MIN, np.array([2, nan, -1], np.float32), None),
        (L.RED_ARGMAX, np.array([nan, 1, 3], np.float32), None),
        (L.RED_ARGMAX, np.array([1, 3, nan, 3], np.float32), None),
        (L.RED_ARGMAX, np.array([nan, nan], np.float32), None),
        (L.RED_ARGMAX, np.array([[nan, 1, 3], [-np.inf, -np.inf, nan], [2, 2, 1]], np.float32), 1),
        (L.RED_ARGMAX, np.array([[nan, 1, 3], [-np.inf, -np.inf, nan], [2, 2, 1]], np.float32), 0),
    ]
    big = np.zeros(300000, np.float32)
    big[[7, 150000, 299999]] = 5.0  # ties across blocks keep the first
    cases.append((L.RED_ARGMAX, big, None))
    for kind, x, axis in cases:
        want = O.reduction(kind, x, axis)
        out = c.empty(want.shape)
        c.reduction(kind, c.to_device(x), axis, out)
        assert_bits(out.numpy(), want, f"{kind} {x.shape} axis {axis}")


def test_kats_through_the_gpu(hip_ctx):  # ops_reduction_complex.rs:5-46, ops_elementwise.rs:6-23
    c = hip_ctx
    a, b = c.to_device(np.array([10.0, 20.0], np.float32)), c.to_device(np.array([2.0, 5.0], np.float32))
    o = c.empty((2,))
    for kind, want in [(L.EW_ADD, [12, 25]), (L.EW_SUB, [8, 15]), (L.EW_MUL, [20, 100]),
                       (L.EW_DIV, [5, 4])]:
        c.elementwise(kind, a, b, o)
        assert o.numpy().tolist() == want
    v = c.empty((1,))
    c.reduction(L.RED_VARIANCE, c.to_device(np.array([2, 4, 4, 4, 5, 5, 7, 9], np.float32)), None, v)
    assert v.numpy()[0] == 4.0
    x = c.to_device(np.array([[1, 5, 2], [9, 3, 4]], np.float32))
    i0, i1 = c.empty((3,)), c.empty((2,))
    c.reduction(L.RED_ARGMAX, x, 0, i0)
    c.reduction(L.RED_ARGMAX, x, 1, i1)
    assert i0.numpy().tolist() == [1.0, 0.0, 1.0] and i1.numpy().tolist() == [1.0, 0.0]
