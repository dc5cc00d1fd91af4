"""Pins of the oracle's axis reductions and axis softmax (CPU only).

The reference reduces an axis with a sequential fp32 loop per output
(backend/cpu/scalar.rs:584-788); it has no axis softmax (ops/stats/softmax.rs:13-16),
so the oracle's float64 axis softmax is pinned against the already-pinned row
softmax with the axis moved last, and its backward by finite differences."""
import numpy as np
import pytest

from oracle import oracle as O

SHAPES_AXES = [((5,), 0), ((3, 4), 0), ((3, 4), 1), ((2, 3, 4), 0), ((2, 3, 4), 1),
               ((2, 3, 4), 2), ((4, 1, 6), 1), ((3, 7, 2, 5), 2)]


@pytest.mark.parametrize("shape,axis", SHAPES_AXES)
def test_reduce_axis_exact_on_integers(shape, axis):
    rng = np.random.default_rng(1)
    x = rng.integers(-50, 50, shape).astype(np.float32)
    want = x.astype(np.float64).sum(axis)
    got = O.reduce_axis(x, axis)
    assert got.shape == (want.shape if want.shape else (1,))
    assert np.array_equal(got.ravel(), want.ravel().astype(np.float32))
    n = np.float32(shape[axis])
    assert np.array_equal(O.reduce_axis(x, axis, mean=True).ravel(),
                          (want.ravel().astype(np.float32) / n).astype(np.float32))


@pytest.mark.parametrize("shape,axis", SHAPES_AXES)
def test_reduce_axis_then_rest_is_full_sum(shape, axis):
    rng = np.random.default_rng(2)
    x = rng.standard_normal(shape).astype(np.float32)
    part = O.reduce_axis(x, axis).astype(np.float64).sum()
    assert abs(part - x.astype(np.float64).sum()) <= 1e-5 * np.abs(x).sum()


def test_reduce_axis_sequential_order():
    """Sequential fp32 accumulation in axis order: 1e8 + 1 + 1 - 1e8 is 0 in that order."""
    x = np.array([[1e8], [1.0], [1.0], [-1e8]], np.float32)
    assert O.reduce_axis(x, 0)[0] == np.float32(0.0)


@pytest.mark.parametrize("shape,axis", SHAPES_AXES)
@pytest.mark.parametrize("mean", [False, True])
def test_broadcast_axis_is_the_gradient(shape, axis, mean):
    """L(x) = sum(g * reduce(x, axis)) is linear, so L(x + v) - L(x) = sum(v * dx) exactly
    in float64 for dx the gradient; a wrong index mapping fails it."""
    rng = np.random.default_rng(3)
    gshape = O.reduce_axis(np.zeros(shape, np.float32), axis).shape
    g = rng.standard_normal(gshape).astype(np.float32)
    dx = O.broadcast_axis(g, shape, axis, mean=mean).astype(np.float64)
    red = (lambda a: a.mean(axis)) if mean else (lambda a: a.sum(axis))
    for _ in range(3):
        v = rng.standard_normal(shape)
        lhs = float((g.astype(np.float64).reshape(-1) * red(v).reshape(-1)).sum())
        rhs = float((v * dx).sum())
        assert abs(lhs - rhs) <= 1e-5 * (abs(lhs) + 1)


@pytest.mark.parametrize("shape,axis", SHAPES_AXES)
def test_softmax_axis_matches_rows_with_axis_last(shape, axis):
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(shape) * 3).astype(np.float32)
    got = O.softmax_axis(x, axis)
    moved = np.ascontiguousarray(np.moveaxis(x, axis, -1))
    rows = O.softmax_rows(moved.reshape(-1, shape[axis])).reshape(moved.shape)
    assert np.array_equal(got, np.moveaxis(rows, -1, axis))
    assert np.allclose(got.astype(np.float64).sum(axis), 1.0, atol=1e-6)


@pytest.mark.parametrize("shape,axis", SHAPES_AXES)
def test_softmax_axis_backward_finite_differences(shape, axis):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(shape).astype(np.float64)
    g = rng.standard_normal(shape).astype(np.float32)

    def sm(a):
        e = np.exp(a - a.max(axis=axis, keepdims=True))
        return e / e.sum(axis=axis, keepdims=True)

    y = O.softmax_axis(x.astype(np.float32), axis)
    dx = O.softmax_axis_backward(y, g, axis).astype(np.float64)
    h = 1e-6
    for _ in range(3):
        v = rng.standard_normal(shape)
        fd = ((g * sm(x + h * v)).sum() - (g * sm(x - h * v)).sum()) / (2 * h)
        assert abs(fd - (v * dx).sum()) <= 1e-4 * (abs(fd) + 1)
    moved_y = np.ascontiguousarray(np.moveaxis(y, axis, -1)).reshape(-1, shape[axis])
    moved_g = np.ascontiguousarray(np.moveaxis(g, axis, -1)).reshape(-1, shape[axis])
    rows = O.softmax_backward(moved_y, moved_g, f64=True)
    back = np.moveaxis(rows.reshape(np.moveaxis(y, axis, -1).shape), -1, axis)
    assert np.array_equal(dx.astype(np.float32), back)
