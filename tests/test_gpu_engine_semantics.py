"""Engine semantics beyond the per-op formulas, on the GPU, through the tensor
API:

* reshape / flatten backward (backward.rs:315-330): the write branch (the
  input's grad cell is empty) and the accumulate branch (one tensor reshaped
  twice), against the oracle's reshape_backward;
* reshape and detach return copies of the values (ops/shape/reshape.rs:103,
  tensor.rs:146-154), so an optimizer step on the source leaves them alone;
* one tensor in two input slots of a node (its grad cell shared,
  tensor.rs:18-33, 120-132): LSTM with W_ih = W_hh, LayerNorm with
  gamma = beta, attention with q = k = v;
* attention with a single head (B = H = 1) where dQ or dK alone is needed,
  whose products split their reduction.
"""
import numpy as np
import pytest

import numrs_amd as nr
from numrs_amd import Tensor, optim
from oracle import oracle as O
from oracle import lstm_oracle as LO
from oracle import transformer_oracle as TO
from tests.conftest import assert_bits, assert_close, assert_contraction, rand

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def ctx(hip_ctx):
    nr.set_default_context(hip_ctx)
    nr.set_unbroadcast_mode("correct")
    yield hip_ctx


# --- a22: reshape / flatten backward ---------------------------------------------

# (in shape, reshaped shape): tiny, a float4-aligned matrix, and one past the
# 2^23-element streaming threshold with a ragged tail.
RESHAPES = [((4, 6), (3, 8)), ((1024, 4096), (4096, 1024)), ((3, (1 << 22) + 5), ((1 << 22) + 5, 3))]


@pytest.mark.parametrize("xs,ys", RESHAPES, ids=["tiny", "4M", "12M_ragged"])
def test_reshape_backward_write_branch(xs, ys):
    print(f"[gpu] reshape write {xs}->{ys}", flush=True)
    rng = np.random.default_rng(22)
    x0, w = rand(rng, xs), rand(rng, ys)
    x = Tensor.new(x0, True)
    y = x.reshape(ys)
    assert y.shape() == ys
    assert_bits(y.values(), x0.reshape(ys), "reshape values")
    loss = y.mul(Tensor.new(w, False)).sum()
    loss.backward()
    g_y = O.mul_backward(O.sum_backward(1.0, ys), x0.reshape(ys), w)[0]
    assert_bits(x.gradient(), O.reshape_backward(g_y, xs), "dx (write branch)")


@pytest.mark.parametrize("xs,ys", RESHAPES, ids=["tiny", "4M", "12M_ragged"])
def test_reshape_backward_accumulate_branch(xs, ys):
    print(f"[gpu] reshape accumulate {xs}->{ys}", flush=True)
    rng = np.random.default_rng(23)
    x0, w1, w2 = rand(rng, xs), rand(rng, ys), rand(rng, xs[::-1])
    x = Tensor.new(x0, True)
    y1 = x.reshape(ys)                      # the same tensor reshaped twice:
    y2 = x.reshape(xs[::-1])                # its grad cell takes two producers
    loss = y1.mul(Tensor.new(w1, False)).sum().add(y2.mul(Tensor.new(w2, False)).sum())
    loss.backward()
    g1 = O.mul_backward(O.sum_backward(1.0, ys), x0.reshape(ys), w1)[0]
    g2 = O.mul_backward(O.sum_backward(1.0, xs[::-1]), x0.reshape(xs[::-1]), w2)[0]
    # accumulate_gradient (tensor.rs:120-132): the second grad adds into the first
    want = O.reshape_backward(g1, xs)
    O.accumulate(want, O.reshape_backward(g2, xs))
    assert_bits(x.gradient(), want, "dx (accumulate branch)")


def test_reshape_of_a_reshape_and_infer():
    rng = np.random.default_rng(24)
    x0, w = rand(rng, (6, 10)), rand(rng, (3, 4, 5))
    x = Tensor.new(x0, True)
    y = x.reshape((4, -1)).reshape((3, 4, -1))      # ops::reshape infers the -1
    assert y.shape() == (3, 4, 5)
    y.mul(Tensor.new(w, False)).sum().backward()
    assert_bits(x.gradient(), O.reshape_backward(w, (6, 10)), "dx through two reshapes")
    for bad in ((7, -1), (-1, -1), (5, 5), (-2, 30)):
        with pytest.raises(nr.HipError):
            x.reshape(bad)


def test_flatten_backward():
    rng = np.random.default_rng(25)
    xs = (2, 3, 4, 5)
    x0 = rand(rng, xs)
    for start, end in ((1, 2), (0, 3), (2, 99), (0, 0)):
        x = Tensor.new(x0, True)
        fs = O.flatten_shape(xs, start, end)
        y = x.flatten(start, end)
        assert y.shape() == fs
        w = rand(rng, fs)
        y.mul(Tensor.new(w, False)).sum().backward()
        assert_bits(x.gradient(), O.reshape_backward(w, xs), f"flatten({start},{end})")
    with pytest.raises(ValueError):
        Tensor.new(x0, True).flatten(3, 1)


def test_reshape_and_detach_copy_the_values():
    rng = np.random.default_rng(26)
    p0, xin = rand(rng, (8, 16)), rand(rng, (8, 16))
    w = Tensor.new(p0, True)
    r = w.reshape((16, 8))
    d = w.detach()
    assert not d.requires_grad and d.is_leaf
    w.mul(Tensor.new(xin, False)).sum().backward()
    opt = optim.SGD([w], 0.1)
    opt.step()
    want = p0.copy()
    O.sgd_step(want, O.mul_backward(O.sum_backward(1.0, (8, 16)), p0, xin)[0], None, 0.1)
    assert_bits(w.values(), want, "param after the step")
    assert_bits(d.values(), p0, "detached copy")               # unchanged by the step
    assert_bits(r.values(), p0.reshape(16, 8), "reshaped copy")
    # prev = w.detach(); opt.step(); w - prev is the update
    assert_bits(w.values() - d.values(), want - p0, "w - prev")


# --- one tensor in two input slots ------------------------------------------------

def test_lstm_with_shared_input_and_recurrent_weight():
    # I == H and W_ih is W_hh: the grad cell receives dW_ih + dW_hh.
    B, T, H = 4, 5, 8
    rng = np.random.default_rng(27)
    x0 = rand(rng, (B, T, H), 0.5)
    w0 = rand(rng, (4 * H, H), 0.3)
    b0 = rand(rng, 4 * H, 0.1)
    dh = rand(rng, (B, T, H))
    x, wt, bt = Tensor.new(x0, True), Tensor.new(w0, True), Tensor.new(b0, True)
    h = x.lstm(wt, wt, bt)
    h.mul(Tensor.new(dh, False)).sum().backward()
    x64, w64 = x0.astype(np.float64), w0.astype(np.float64)
    hs, cache = LO.lstm_layer(x64, w64, w64, b0.astype(np.float64))
    dx, dwi, dwh, db = LO.lstm_layer_backward(x64, w64, w64, hs, cache, dh.astype(np.float64))
    assert_close(h.values(), hs, what="h")
    assert_contraction(wt.gradient(), dwi + dwh, 2 * B * T, what="dW (shared)")
    assert_contraction(x.gradient(), dx, 4 * H, what="dx")
    assert_contraction(bt.gradient(), db, B * T, what="db")


def test_layernorm_with_gamma_as_beta():
    R, C = 64, 96
    rng = np.random.default_rng(28)
    x0, g0 = rand(rng, (R, C)), rand(rng, (R, C))
    gb0 = rng.uniform(0.5, 1.5, C).astype(np.float32)
    x, gb = Tensor.new(x0, True), Tensor.new(gb0, True)
    y = x.layer_norm(gb, gb)
    y.mul(Tensor.new(g0, False)).sum().backward()
    dx, dgamma, dbeta = O.layernorm_backward(g0, x0, gb0)
    assert_close(x.gradient(), dx, what="dx")
    assert_close(gb.gradient(), dgamma.astype(np.float64) + dbeta, abs_tol=1e-5 + 2e-7 * R,
                 what="dgamma + dbeta")


@pytest.mark.parametrize("S", [128, 256])
@pytest.mark.parametrize("mode", ["dq", "dk", "dv", "self"])
def test_attention_single_head(S, mode):
    """B = H = 1, dh = 64: dQ = dS K and dK = dS^T Q are single 128 x 64 or
    256 x 64 products with an S-long reduction, which split it (the split
    partials must not overwrite dS)."""
    print(f"[gpu] attention single head S={S} mode={mode}", flush=True)
    D = 64
    rng = np.random.default_rng(29 + S)
    q0, k0, v0, w = (rand(rng, (S, D)) for _ in range(4))
    if mode == "self":
        xt = Tensor.new(q0, True)
        q = k = v = xt
        k0 = v0 = q0
    else:
        q = Tensor.new(q0, mode == "dq")
        k = Tensor.new(k0, mode == "dk")
        v = Tensor.new(v0, mode == "dv")
    o = q.attention(k, v, 1, S, 1)
    o.mul(Tensor.new(w, False)).sum().backward()
    out, cache = TO.attention_forward(*(a.astype(np.float64) for a in (q0, k0, v0)), 1, S, 1)
    dq, dk, dv = TO.attention_backward(w.astype(np.float64), cache, 1, S, 1)
    assert_contraction(o.values(), out, S, what="out")
    if mode == "self":
        assert_contraction(xt.gradient(), dq + dk + dv, S + D, what="dx (q = k = v)")
        return
    got = {"dq": q, "dk": k, "dv": v}[mode].gradient()
    assert_contraction(got, {"dq": dq, "dk": dk, "dv": dv}[mode], S + D, what=mode)
    for name, t in (("dq", q), ("dk", k), ("dv", v)):
        if name != mode:
            assert t.gradient() is None, name


@pytest.mark.parametrize("loss_kind", ["mse", "ce", "ce_labels"])
@pytest.mark.parametrize("input_grad", [True, False])
def test_loss_root_seed(hip_ctx, loss_kind, input_grad):
    """backward() seeds the root's gradient with ones (tensor.rs:178-183).  A
    scalar MSE / cross-entropy root has the seed written by its own backward
    kernel; when that kernel does not run (the input needs no gradient) the
    seed is still written."""
    print(f"[gpu] loss seed {loss_kind} input_grad={input_grad}", flush=True)
    if loss_kind == "ce_labels" and not input_grad:
        pytest.skip("labels carry no gradient: the loss would not require one")
    nr.set_default_context(hip_ctx)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((6, 5)).astype(np.float32)
    xt = Tensor.new(x, input_grad)
    if loss_kind == "mse":
        t = rng.standard_normal((6, 5)).astype(np.float32)
        loss = xt.mse_loss(Tensor.new(t, True))
        want_x = (2.0 * (x.astype(np.float64) - t)) / x.size
    else:
        lab = rng.integers(0, 5, 6)
        if loss_kind == "ce":
            # a one-hot target that requires grad keeps the loss recorded when
            # the logits do not (its gradient is the reference's [0])
            loss = xt.cross_entropy_loss(Tensor.new(np.eye(5, dtype=np.float32)[lab],
                                                    not input_grad))
        else:
            loss = xt.cross_entropy_labels(lab)
        e = np.exp(x - x.max(1, keepdims=True))
        want_x = (e / e.sum(1, keepdims=True) - np.eye(5)[lab]) / 6
    loss.backward()
    assert loss.gradient().tolist() == [1.0]
    if input_grad:
        assert_close(xt.gradient(), want_x, abs_tol=1e-7, rel_tol=1e-5, what="input grad")
    # a second backward accumulates (the seed is 1 again, the input grad doubles)
    if input_grad:
        first = xt.gradient().copy()
        loss.backward()
        assert loss.gradient().tolist() == [1.0]
        assert_close(xt.gradient(), 2 * first, abs_tol=1e-7, rel_tol=1e-6, what="accumulated")


@pytest.mark.parametrize("loss_kind", ["mse", "mse_large", "ce", "ce_labels"])
def test_preformed_loss_gradient_equals_backward_kernel(hip_ctx, loss_kind):
    """A scalar loss whose input needs a gradient forms the gradient its
    backward would form as the root (and the root's seed) in its forward
    kernel; backward() then adopts it.  It equals the backward kernel's
    result bit for bit: the same loss reached through a Mul by 1 (so it is no
    longer the root) runs that kernel with g = 1.  The root's gradient is 1
    even after set_gradient / zero_grad on it between forward and backward."""
    print(f"[gpu] pre-formed loss gradient {loss_kind}", flush=True)
    nr.set_default_context(hip_ctx)
    rng = np.random.default_rng(11)
    shape = (4096, 512) if loss_kind == "mse_large" else (64, 10)
    x = rng.standard_normal(shape).astype(np.float32)
    t = rng.standard_normal(shape).astype(np.float32)
    lab = rng.integers(0, shape[1], shape[0])
    onehot = np.eye(shape[1], dtype=np.float32)[lab]

    def loss_of(xt):
        if loss_kind.startswith("mse"):
            return xt.mse_loss(Tensor.new(t, False))
        if loss_kind == "ce":
            return xt.cross_entropy_loss(Tensor.new(onehot, False))
        return xt.cross_entropy_labels(lab)

    xa = Tensor.new(x, True)
    la = loss_of(xa)
    la.backward()
    assert la.gradient().tolist() == [1.0]
    xb = Tensor.new(x, True)
    lb = loss_of(xb).mul(Tensor.new(np.ones(1, np.float32), False))
    lb.backward()
    assert np.array_equal(xa.gradient(), xb.gradient())
    # the root's cell written between forward and backward: the seed is still 1
    xc = Tensor.new(x, True)
    lc = loss_of(xc)
    lc.set_gradient(np.array([5.0], np.float32))
    lc.zero_grad()
    lc.backward()
    assert lc.gradient().tolist() == [1.0]
    assert np.array_equal(xc.gradient(), xa.gradient())
