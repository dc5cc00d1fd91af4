"""The streaming access mode (non-temporal float4 loads and stores, taken by
arrays of at least 2^23 floats) of every kernel that has one, against the
oracle at sizes just past the threshold.  Element counts are ragged where
the shape allows, so the last block mixes the vector path with the
per-element tail.  The kernels' arithmetic is the same in both modes, so
the bars are those of the cached-mode tests: bit-exact where the oracle is
fp32-faithful, the north-star tolerance (plus the length-n sum allowance)
for reductions.
"""
from __future__ import annotations

import numpy as np
import pytest

from numrs_amd import _lib as L
from oracle import oracle as O
from tests.conftest import assert_bits, assert_close, assert_sum, rand

pytestmark = pytest.mark.gpu

N = (1 << 23) + 3  # past the streaming threshold, with a 3-element tail


@pytest.fixture()
def rng():
    return np.random.default_rng(20261202)


def say(msg):
    print(f"[gpu] {msg}", flush=True)


@pytest.mark.parametrize("kind,name", [(L.RELU, "relu"), (L.TANH, "tanh")])
def test_unary_backward_streaming(hip_ctx, rng, kind, name):
    say(f"unary_backward {name} n={N}")
    g, x = rand(rng, N), rand(rng, N)
    x[:7] = 0.0  # the strict mask at zero
    c = hip_ctx
    v = x if kind == L.RELU else np.tanh(x).astype(np.float32)
    dx = c.empty((N,))
    c.unary_backward(kind, c.to_device(g), c.to_device(v), dx)
    want = O.relu_backward(g, v) if kind == L.RELU else O.tanh_backward(g, v)
    assert_bits(dx.numpy(), want, name)


def test_binary_mul_backward_streaming(hip_ctx, rng):
    say(f"binary_backward mul n={N}")
    g, x, y = rand(rng, N), rand(rng, N), rand(rng, N)
    c = hip_ctx
    dx, dy = c.empty((N,)), c.empty((N,))
    c.binary_backward(L.MUL, c.to_device(g), c.to_device(x), c.to_device(y), dx, dy)
    wx, wy = O.mul_backward(g, x, y)
    assert_bits(dx.numpy(), wx, "dx")
    assert_bits(dy.numpy(), wy, "dy")


def test_fill_mse_sgd_streaming(hip_ctx, rng):
    say(f"fill_grad, mse_backward, sgd_step n={N}")
    c = hip_ctx
    g1 = c.to_device(np.array([0.75], np.float32))
    dx = c.empty((N,))
    c.fill_grad(g1, dx, divide_by_n=True)
    assert_bits(dx.numpy(), O.mean_backward(0.75, (N,)), "fill")
    p, t = rand(rng, N), rand(rng, N)
    dp = c.empty((N,))
    c.mse_backward(g1, c.to_device(p), c.to_device(t), dp)
    assert_bits(dp.numpy(), O.mse_backward(0.75, p, t)[0], "mse dp")
    for mu, wd in ((0.0, 0.0), (0.9, 0.01)):
        pp, gg = rand(rng, N), rand(rng, N)
        vv = rand(rng, N, 0.1)
        pd, vd = c.to_device(pp), c.to_device(vv)
        c.sgd_step(pd, c.to_device(gg), vd if mu else None, lr=0.01, mu=mu, wd=wd)
        O.sgd_step(pp, gg, vv if mu else None, 0.01, mu=mu, wd=wd)
        assert_bits(pd.numpy(), pp, f"sgd p mu={mu}")
        if mu:
            assert_bits(vd.numpy(), vv, "sgd v")


def test_row_kernels_streaming(hip_ctx, rng):
    # [8192, 1024] = 2^23 elements: softmax-CE, softmax backward, argmax rows
    R, C = 8192, 1024
    say(f"softmax_ce_backward, softmax_backward, argmax [{R},{C}]")
    c = hip_ctx
    logits = rand(rng, (R, C), 2.0)
    lab = rng.integers(0, C, R)
    onehot = np.zeros((R, C), np.float32)
    onehot[np.arange(R), lab] = 1.0
    g1 = c.to_device(np.array([0.75], np.float32))
    dl = c.empty((R, C))
    c.softmax_ce_backward(g1, c.to_device(logits), dl, onehot=c.to_device(onehot))
    assert_close(dl.numpy()[:256], O.cross_entropy_backward(0.75, logits[:256], onehot[:256]) *
                 np.float32(256 / R), what="ce")
    y = O.softmax_rows(logits)
    gs = rand(rng, (R, C))
    ds = c.empty((R, C))
    c.softmax_backward(c.to_device(y), c.to_device(gs), ds)
    assert_close(ds.numpy()[:512], O.softmax_backward(y[:512], gs[:512], f64=True),
                 what="softmax bwd")
    idx = c.empty((R,), np.int32)
    c.argmax_rows(c.to_device(logits), idx)
    assert np.array_equal(idx.numpy(), O.argmax_rows(logits)), "argmax"


def test_sums_transpose_layernorm_streaming(hip_ctx, rng):
    c = hip_ctx
    say(f"sum n={N}, sum_to_shape [8192,1024], transpose [2048,4096], layernorm [16384,512]")
    # Device arrays are held in variables for the whole call: a temporary's
    # memory is released as soon as its pointer has been read.
    x = rand(rng, N)
    xd, s = c.to_device(x), c.empty((1,))
    c._check(L.load().numrs_hip_sum(c.handle, xd.ptr, N, 0, s.ptr))
    assert_sum(s.numpy(), [x.astype(np.float64).sum()], N, what="full sum")
    gm = rand(rng, (8192, 1024))
    b = c.empty((1024,))
    c.sum_to_shape(c.to_device(gm), b)
    assert_sum(b.numpy(), gm.astype(np.float64).sum(0), 8192, what="column sum")
    tm = rand(rng, (2048, 4096))
    tmd, tr = c.to_device(tm), c.empty((4096, 2048))
    c._check(L.load().numrs_hip_transpose(c.handle, tmd.ptr, tr.ptr, 2048, 4096))
    assert_bits(tr.numpy(), O.transpose(tm), "transpose")
    RL = 16384
    xl, gl = rand(rng, (RL, 512)), rand(rng, (RL, 512))
    gam = (1.0 + 0.1 * rng.standard_normal(512)).astype(np.float32)
    _, mean, rstd = O.layernorm_fwd(xl, gam, np.zeros(512, np.float32))
    gd, xd, gamd, md, rd = (c.to_device(a) for a in (gl, xl, gam, mean, rstd))
    dxl, dg, db = c.empty((RL, 512)), c.empty((512,)), c.empty((512,))
    c._check(L.load().numrs_hip_layernorm_backward(
        c.handle, gd.ptr, xd.ptr, gamd.ptr, md.ptr, rd.ptr, dxl.ptr, dg.ptr, db.ptr, RL, 512,
        0, 0, 0))
    wdx, wdg, wdb = O.layernorm_backward(gl[:2048], xl[:2048], gam)
    assert_close(dxl.numpy()[:2048], wdx, abs_tol=1e-5, rel_tol=1e-4, what="ln dx")
    assert_sum(db.numpy(), gl.astype(np.float64).sum(0), RL, what="ln dbeta")


@pytest.mark.parametrize("n", [4096 + 4, 1 << 23], ids=["cached", "streaming"])
@pytest.mark.parametrize("reads,writes", [(0, 1), (1, 0), (1, 1), (1, 2), (2, 1), (3, 2)])
def test_stream_probe(hip_ctx, rng, n, reads, writes):
    """numrs_hip_stream_probe (the bench's ceiling for the streaming rows):
    y (and z) = (a + b) + c over the first `reads` operands, zeros for none;
    nothing stored for writes = 0; bad arguments refused."""
    say(f"stream_probe reads={reads} writes={writes} n={n}")
    c = hip_ctx
    ops = [rand(rng, n) for _ in range(3)]
    dev = [c.to_device(a) for a in ops]
    y = c.to_device(np.full(n, 7.0, np.float32))
    z = c.to_device(np.full(n, 7.0, np.float32))
    ptr = [d.ptr if i < reads else None for i, d in enumerate(dev)]
    c._check(L.load().numrs_hip_stream_probe(c.handle, ptr[0], ptr[1], ptr[2], y.ptr,
                                             z.ptr if writes == 2 else None, n, reads, writes))
    used = [a if i < reads else np.zeros(n, np.float32) for i, a in enumerate(ops)]
    want = (used[0] + used[1]) + used[2]
    if writes == 0:
        assert np.array_equal(y.numpy(), np.full(n, 7.0, np.float32))
    else:
        assert_bits(y.numpy(), want)
    assert_bits(z.numpy(), want if writes == 2 else np.full(n, 7.0, np.float32))
    from numrs_amd import HipError
    with pytest.raises(HipError):
        c._check(L.load().numrs_hip_stream_probe(c.handle, ptr[0], ptr[1], ptr[2], y.ptr,
                                                 None, n + 2, reads, writes))
