"""Axis reductions and axis softmax on the GPU, against the oracle.

numrs's ops::sum / ops::mean reduce one axis with a sequential fp32 loop per
output (backend/cpu/scalar.rs:584-788); its autograd only ever reduces fully and
its sum_backward ignores the axis (backward.rs:208-221), and ops::softmax
rejects an axis (ops/stats/softmax.rs:13-16).  These are the upstream-compatible
fixes: forward values within fp32 tolerance of the sequential loop, gradients
against the oracle's broadcast / float64 softmax backward."""
import numpy as np
import pytest

import numrs_amd as nr
from numrs_amd import Tensor
from numrs_amd import _lib as L
from oracle import oracle as O
from tests.conftest import assert_bits, assert_close, rand

pytestmark = pytest.mark.gpu

CASES = [((5,), 0), ((3, 4), 0), ((3, 4), 1), ((2, 3, 4), 0), ((2, 3, 4), 1), ((2, 3, 4), 2),
         ((7, 1000, 3), 1), ((4096, 64), 0), ((64, 4096), 1), ((16, 8, 256), 1),
         ((3, 5, 2, 7), 2)]


def say(msg):
    print(f"[gpu-axis] {msg}", flush=True)


@pytest.fixture(scope="module", autouse=True)
def ctx(hip_ctx):
    nr.set_default_context(hip_ctx)
    yield hip_ctx


@pytest.mark.parametrize("shape,axis", CASES)
@pytest.mark.parametrize("mean", [0, 1])
def test_reduce_and_broadcast_axis(hip_ctx, shape, axis, mean):
    say(f"reduce_axis {shape} axis={axis} mean={mean}")
    rng = np.random.default_rng(10)
    x = rand(rng, shape)
    o, n, i = O.axis_view(shape, axis)
    c = hip_ctx
    xd = c.to_device(x)
    out = c.empty((o * i,))
    c._check(L.load().numrs_hip_reduce_axis(c.handle, xd.ptr, o, n, i, mean, out.ptr))
    want = O.reduce_axis(x, axis, mean=bool(mean)).ravel()
    tol = 1e-5 + 2e-7 * n  # a length-n fp32 sum in another order
    assert_close(out.numpy(), x.astype(np.float64).sum(axis).ravel() / (n if mean else 1),
                 abs_tol=tol, what="vs float64")
    assert_close(out.numpy(), want, abs_tol=2 * tol, what="vs numrs loop")
    g = rand(rng, (o * i,))
    dx, gd = c.empty(shape), c.to_device(g)  # held for the call: a temporary is freed at once
    c._check(L.load().numrs_hip_broadcast_axis(c.handle, gd.ptr, o, n, i, mean, dx.ptr, 0))
    assert_bits(dx.numpy(), O.broadcast_axis(g, shape, axis, mean=bool(mean)), "broadcast")


def test_reduce_axis_empty_axis(hip_ctx):
    c = hip_ctx
    out = c.empty((6,))
    x = c.empty((1,))
    c._check(L.load().numrs_hip_reduce_axis(c.handle, x.ptr, 2, 0, 3, 0, out.ptr))
    assert np.all(out.numpy() == 0)
    c._check(L.load().numrs_hip_reduce_axis(c.handle, x.ptr, 2, 0, 3, 1, out.ptr))
    assert np.all(np.isnan(out.numpy()))


@pytest.mark.parametrize("shape,axis", CASES)
def test_softmax_axis_forward_backward(hip_ctx, shape, axis):
    say(f"softmax_axis {shape} axis={axis}")
    rng = np.random.default_rng(11)
    x = rand(rng, shape, 3.0)
    g = rand(rng, shape)
    o, n, i = O.axis_view(shape, axis)
    c = hip_ctx
    y, xd = c.empty(shape), c.to_device(x)  # held for the call: a temporary is freed at once
    c._check(L.load().numrs_hip_softmax_axis_forward(c.handle, xd.ptr, y.ptr, o, n, i))
    want_y = O.softmax_axis(x, axis)
    assert_close(y.numpy(), want_y, what="softmax")
    yd = c.to_device(want_y)
    dx = c.to_device(np.ones(shape, np.float32))
    gd = c.to_device(g)
    c._check(L.load().numrs_hip_softmax_axis_backward(c.handle, yd.ptr, gd.ptr, dx.ptr, o, n, i,
                                                       1))
    assert_close(dx.numpy(), 1.0 + O.softmax_axis_backward(want_y, g, axis).astype(np.float64),
                 what="softmax backward (accumulate)")


@pytest.mark.parametrize("shape,axis", [((3, 4), 0), ((2, 3, 4), 1), ((16, 8, 256), 2),
                                        ((64, 4096), 1), ((4096, 64), 0)])
def test_tensor_axis_ops_autograd(shape, axis):
    """Tensor.sum/mean/softmax with an axis through the engine: values and grads.
    x feeds two branches, so its grad cell also accumulates."""
    rng = np.random.default_rng(12)
    X = rand(rng, shape)
    x = Tensor.new(X, True)
    s = x.sum(axis)
    m = x.mean(axis)
    sm = x.softmax(axis)
    assert s.shape() == O.reduce_axis(X, axis).shape
    o, n, i = O.axis_view(shape, axis)
    tol = 1e-5 + 2e-7 * n
    assert_close(s.values(), X.astype(np.float64).sum(axis).reshape(s.shape()), abs_tol=tol)
    assert_close(m.values(), X.astype(np.float64).mean(axis).reshape(m.shape()), abs_tol=tol)
    Y = O.softmax_axis(X, axis)
    assert_close(sm.values(), Y, what="softmax values")
    ws, wm, wy = rand(rng, s.shape()), rand(rng, m.shape()), rand(rng, shape)
    loss = (s.mul(Tensor.new(ws, False)).sum()
            .add(m.mul(Tensor.new(wm, False)).sum())
            .add(sm.mul(Tensor.new(wy, False)).sum()))
    loss.backward()
    want = (O.broadcast_axis(ws, shape, axis).astype(np.float64)
            + O.broadcast_axis(wm, shape, axis, mean=True)
            + O.softmax_axis_backward(sm.values(), wy, axis))
    assert_close(x.gradient(), want, what="grad")


def test_tensor_axis_errors():
    x = Tensor.new(np.ones((2, 3), np.float32), True)
    with pytest.raises(ValueError):
        x.sum(2)
    with pytest.raises(ValueError):
        x.softmax(-3)
    assert x.sum(-1).shape() == (2,)
    assert Tensor.new(np.ones(4, np.float32), True).sum(0).shape() == (1,)
