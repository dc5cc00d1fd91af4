"""Split-K partials added inside the products' own launch (the default,
numrs_hip_set_split_reduction FUSED, for the 128 x 64 streamed tiles and the
16 x 16 tiny blocks) against one more launch after them (SEPARATE): the same
bits, for the Linear backward pairs of the C4 block, for matmul_backward
shapes whose weight-side product splits, for C1's first layer, and for the
C5 forecaster's paired LSTM weight gradients.  (Products
on the 256 x 128 tiles keep the separate launch in both modes.)  The fused
form's arrival counters are reset by the launches themselves, so
back-to-back calls and replays of a recorded graph must each be whole."""
import numpy as np
import pytest

import numrs_amd as nr
from numrs_amd import StepGraph, Tensor, nn
from numrs_amd import _lib as L
from oracle import lstm_oracle as LO

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rng():
    return np.random.default_rng(2024)


def _linear_bwd(c, gd, xd, Wd, outs, T, fin, fout, acc):
    dx, dW, db = outs
    rc = L.load().numrs_hip_linear_backward(c.handle, gd.ptr, xd.ptr, Wd.ptr, dx.ptr, dW.ptr, db.ptr,
                                            T, fin, fout, *acc, L.UNBROADCAST_CORRECT)
    assert rc == 0


# The C4 block's four Linear shapes (all split their weight gradient; the
# packed q/k/v projection splits dx too), a small-tile product and a shape
# whose bias columns end on a partial column group.
@pytest.mark.parametrize("T,fin,fout", [(4096, 2048, 512), (4096, 512, 2048), (4096, 512, 512),
                                        (4096, 512, 1536), (2048, 256, 256), (8192, 64, 100)])
def test_linear_backward_fused_equals_separate(hip_ctx, rng, T, fin, fout):
    print(f"[gpu] fused split reduction: linear backward T={T} in={fin} out={fout}", flush=True)
    c = hip_ctx
    x = rng.standard_normal((T, fin), dtype=np.float32)
    W = rng.standard_normal((fout, fin), dtype=np.float32)
    prev = [rng.standard_normal(s, dtype=np.float32) for s in ((T, fin), (fout, fin), (fout,))]
    xd, Wd = c.to_device(x), c.to_device(W)
    try:
        for acc in ((0, 0, 0), (1, 1, 1)):
            got = {}
            for mode in ("separate", "fused", "fused"):  # fused twice: counters back at zero
                c.set_split_reduction(mode)
                g = rng.standard_normal((T, fout), dtype=np.float32) if mode == "separate" else g
                gd = c.to_device(g)
                outs = [c.to_device(p) for p in prev]
                _linear_bwd(c, gd, xd, Wd, outs, T, fin, fout, acc)
                vals = [o.numpy() for o in outs]
                if mode in got:
                    for a, b, name in zip(got[mode], vals, ("dx", "dW", "db")):
                        assert np.array_equal(a, b), f"second fused call {name} {acc}"
                got[mode] = vals
            for a, b, name in zip(got["separate"], got["fused"], ("dx", "dW", "db")):
                assert np.array_equal(a, b), f"{name} acc={acc}"
    finally:
        c.set_split_reduction("fused")


# matmul_backward shapes whose dB = A^T dC runs over a long reduction (M):
# the planner cuts it into split-K ranges beside the unsplit dA tiles.
@pytest.mark.parametrize("M,K,N", [(8192, 512, 512), (16384, 256, 512), (4096, 1024, 256)])
def test_matmul_backward_fused_equals_separate(hip_ctx, rng, M, K, N):
    print(f"[gpu] fused split reduction: matmul_backward {M}x{K}x{N}", flush=True)
    c = hip_ctx
    A = c.to_device(rng.standard_normal((M, K), dtype=np.float32))
    B = c.to_device(rng.standard_normal((K, N), dtype=np.float32))
    dC = c.to_device(rng.standard_normal((M, N), dtype=np.float32))
    got = {}
    try:
        for mode in ("separate", "fused"):
            c.set_split_reduction(mode)
            dA, dB = c.empty((M, K)), c.empty((K, N))
            c.matmul_backward(dC, A, B, dA, dB)
            got[mode] = (dA.numpy(), dB.numpy())
    finally:
        c.set_split_reduction("fused")
    assert np.array_equal(got["separate"][0], got["fused"][0]), "dA"
    assert np.array_equal(got["separate"][1], got["fused"][1]), "dB"


# Tiny products (16 x 16 blocks) split over a long reduction: C1's first
# layer (Linear 784 -> 128 over 64 rows, with and without the ReLU epilogue)
# and a plain product with ragged blocks; the block's last split reduces it.
@pytest.mark.parametrize("what", ["linear", "linear_relu", "matmul_ragged"])
def test_tiny_split_fused_equals_separate(hip_ctx, rng, what):
    print(f"[gpu] fused split reduction: tiny {what}", flush=True)
    c = hip_ctx
    lib = L.load()
    if what == "matmul_ragged":
        M, K, N = 37, 3000, 45
        A = c.to_device(rng.standard_normal((M, K), dtype=np.float32))
        B = c.to_device(rng.standard_normal((K, N), dtype=np.float32))
        prev = rng.standard_normal((M, N), dtype=np.float32)

        def run():
            C = c.to_device(prev)
            c.matmul(A, B, C, accumulate=True)
            return C.numpy()
    else:
        T, fin, fout = 64, 784, 128
        x = c.to_device(rng.standard_normal((T, fin), dtype=np.float32))
        W = c.to_device(rng.standard_normal((fout, fin), dtype=np.float32))
        b = c.to_device(rng.standard_normal((fout,), dtype=np.float32))
        fn = lib.numrs_hip_linear_forward if what == "linear" else lib.numrs_hip_linear_relu_forward

        def run():
            y = c.empty((T, fout))
            assert fn(c.handle, x.ptr, W.ptr, b.ptr, y.ptr, T, fin, fout) == 0
            return y.numpy()
    try:
        c.set_split_reduction("separate")
        sep = run()
        c.set_split_reduction("fused")
        first, second = run(), run()  # twice: the counters are back at zero
    finally:
        c.set_split_reduction("fused")
    assert np.array_equal(sep, first)
    assert np.array_equal(sep, second)


def test_lstm_forecaster_fused_equals_separate(hip_ctx, monkeypatch):
    """C5 end to end: the head Linear's split product (tiny blocks) reduces
    in its own launch; the layers' paired weight gradients (a 128 x 64 grid
    that leaves slots free) keep the separate reduce in both modes."""
    print("[gpu] fused split reduction: C5 forecaster", flush=True)
    nr.set_default_context(hip_ctx)
    monkeypatch.setattr(nn.LSTMForecaster, "fuse_stack", True)

    def run(mode):
        hip_ctx.set_split_reduction(mode)
        try:
            layers, hw, hb, x, target = LO.make_c5(seed=17, n_layers=2, B=64, T=128, I=64, H=256)
            model = nn.LSTMForecaster(layers, hw, hb)
            xt = Tensor.new(x, True)
            loss = model.forward(xt).mse_loss(Tensor.new(target, False))
            loss.backward()
            out = {"x": xt.gradient(), "head_w": model.head.weight.gradient()}
            for li, layer in enumerate(model.layers):
                out[f"w_ih{li}"] = layer.w_ih.gradient()
                out[f"w_hh{li}"] = layer.w_hh.gradient()
                out[f"b{li}"] = layer.bias.gradient()
            return out
        finally:
            hip_ctx.set_split_reduction("fused")

    sep, fus = run("separate"), run("fused")
    for name, v in sep.items():
        assert np.array_equal(v, fus[name]), name


def test_fused_linear_backward_graph_replays(hip_ctx, rng):
    """A fused Linear backward (C4's 512 -> 512 layer, small tiles, dW split)
    recorded into a graph: each replay, with new g uploaded and eager fused
    calls of the same shape in between, equals an eager call on the same
    inputs."""
    print("[gpu] fused split reduction: graph replays", flush=True)
    c = hip_ctx
    T, fin, fout = 4096, 512, 512
    x = c.to_device(rng.standard_normal((T, fin), dtype=np.float32))
    W = c.to_device(rng.standard_normal((fout, fin), dtype=np.float32))
    g = c.to_device(rng.standard_normal((T, fout), dtype=np.float32))
    rec = [c.empty((T, fin)), c.empty((fout, fin)), c.empty((fout,))]
    eag = [c.empty((T, fin)), c.empty((fout, fin)), c.empty((fout,))]
    _linear_bwd(c, g, x, W, rec, T, fin, fout, (0, 0, 0))  # every buffer exists before recording
    c.sync()
    graph = StepGraph(c, lambda: _linear_bwd(c, g, x, W, rec, T, fin, fout, (0, 0, 0)))
    try:
        for k in range(4):
            g.upload(rng.standard_normal((T, fout), dtype=np.float32))
            graph.replay()
            _linear_bwd(c, g, x, W, eag, T, fin, fout, (0, 0, 0))
            for a, b, name in zip(rec, eag, ("dx", "dW", "db")):
                assert np.array_equal(a.numpy(), b.numpy()), f"replay {k}: {name}"
    finally:
        graph.close()
