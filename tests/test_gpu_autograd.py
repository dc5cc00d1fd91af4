"""The device autograd engine through numrs's own API, on the GPU.

Known-answer tests are the reference's (file:line cited), run through
numrs_amd.Tensor exactly as the Rust tests call Tensor; the C1 MLP step is
compared with the oracle composition in oracle/mlp_oracle.py.
"""
import numpy as np
import pytest

import numrs_amd as nr
from numrs_amd import Tensor, nn, optim
from oracle import oracle as O
from tests.conftest import assert_close, assert_contraction, rand
from oracle.mlp_oracle import make_c1, mlp_step

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def ctx(hip_ctx):
    nr.set_default_context(hip_ctx)
    nr.set_unbroadcast_mode("correct")
    yield hip_ctx


# --- tests/autograd_basic.rs ---------------------------------------------------

def test_creates_tensor():  # autograd_basic.rs:6-12
    t = Tensor.new([1.0, 2.0, 3.0, 4.0], True, shape=(2, 2))
    assert t.shape() == (2, 2)
    assert t.requires_grad
    assert t.gradient() is not None


def test_backward_add():  # autograd_basic.rs:15-40
    x = Tensor.new([1.0, 2.0], True)
    y = Tensor.new([3.0, 4.0], True)
    z = x.add(y)
    assert z.values().tolist() == [4.0, 6.0]
    z.backward()
    assert x.gradient().tolist() == [1.0, 1.0]
    assert y.gradient().tolist() == [1.0, 1.0]


def test_backward_mul():  # autograd_basic.rs:43-68
    x = Tensor.new([2.0, 3.0], True)
    y = Tensor.new([4.0, 5.0], True)
    z = x.mul(y)
    assert z.values().tolist() == [8.0, 15.0]
    z.backward()
    assert x.gradient().tolist() == [4.0, 5.0]
    assert y.gradient().tolist() == [2.0, 3.0]


def test_complex_graph():  # autograd_basic.rs:71-97
    x = Tensor.new([2.0], True)
    y = Tensor.new([3.0], True)
    z = x.mul(y).add(x)
    assert z.values()[0] == 8.0
    z.backward()
    assert x.gradient()[0] == 4.0
    assert y.gradient()[0] == 2.0


def test_no_grad_tensor():  # autograd_basic.rs:100-117
    x = Tensor.new([1.0], True)
    y = Tensor.new([1.0], False)
    x.add(y).backward()
    assert x.gradient() is not None
    assert y.gradient() is None


def test_no_grad_mode_records_nothing():  # autograd/mod.rs:209-246
    x = Tensor.new([1.0, 2.0], True)
    with nr.no_grad():
        y = x.mul(x)
    assert not y.requires_grad and y.is_leaf
    with pytest.raises(nr.HipError):
        y.backward()  # "Tensor does not require gradients" (tensor.rs:174-176)


# --- tests/autograd_matmul.rs, autograd_activations.rs, autograd_loss.rs, autograd_reduction.rs

def test_matmul_backward_kat():  # autograd_matmul.rs:6-47
    a = Tensor.new([1.0, 2.0, 3.0, 4.0], True, shape=(2, 2))
    b = Tensor.new([1.0, 0.0, 0.0, 1.0], True, shape=(2, 2))
    c = a.matmul(b)
    assert c.values().ravel().tolist() == [1.0, 2.0, 3.0, 4.0]
    c.backward()
    assert a.gradient().ravel().tolist() == [1.0, 1.0, 1.0, 1.0]
    assert b.gradient().ravel().tolist() == [4.0, 4.0, 6.0, 6.0]


def test_relu_backward_kat():  # autograd_activations.rs:5-24
    x = Tensor.new([-1.0, 0.0, 1.0], True)
    y = nn.ReLU().forward(x)
    y.backward()
    g = x.gradient()
    assert g[0] == 0.0 and g[2] == 1.0 and g[1] == 0.0


def test_sigmoid_values():  # autograd_activations.rs:26-37
    y = nn.Sigmoid().forward(Tensor.new([0.0, 2.0, -2.0], False)).values()
    assert y[0] == 0.5 and abs(y[1] - 0.880797) < 1e-5 and abs(y[2] - 0.119202) < 1e-5


def test_softmax_dim():  # autograd_activations.rs:39-51 (ignored in the reference: no axis)
    y = nn.Softmax().forward(Tensor.new([0.0, 0.0], False, shape=(1, 2))).values()
    assert y.ravel().tolist() == [0.5, 0.5]


def test_mse_loss_kat():  # autograd_loss.rs:5-37
    pred = Tensor.new([1.0, 2.0, 3.0], True)
    target = Tensor.new([1.0, 2.0, 5.0], False)
    loss = pred.mse_loss(target)
    assert abs(loss.item() - 1.3333333) < 1e-5
    loss.backward()
    g = pred.gradient()
    assert g[0] == 0.0 and abs(g[2] + 1.333333) < 1e-5


def test_cross_entropy_basic():  # autograd_loss.rs:40-54
    logits = Tensor.new([2.0, -1.0], False, shape=(1, 2))
    targets = Tensor.new([1.0, 0.0], False, shape=(1, 2))
    assert logits.cross_entropy_loss(targets).item() < 0.1


def test_sum_mean_backward():  # autograd_reduction.rs:6-40
    x = Tensor.new([1.0, 2.0, 3.0, 4.0], True, shape=(2, 2))
    s = x.sum()
    assert s.values().tolist() == [10.0]
    s.backward()
    assert x.gradient().ravel().tolist() == [1.0] * 4
    x = Tensor.new([1.0, 2.0, 3.0, 4.0], True)
    m = x.mean()
    assert m.values()[0] == 2.5
    m.backward()
    assert x.gradient().tolist() == [0.25] * 4


# --- tests/autograd/optim/{sgd,adam}.rs ------------------------------------------

def test_sgd_kats():  # sgd.rs:8-80
    p = Tensor.new([1.0, 2.0], True)
    p.set_gradient([0.1, 0.2])
    optim.SGD([p], 0.1, 0.0, 0.0).step()
    v = p.values()
    assert abs(v[0] - 0.99) < 1e-5 and abs(v[1] - 1.98) < 1e-5
    p = Tensor.new([1.0], True)
    p.set_gradient([1.0])
    o = optim.SGD([p], 0.1, 0.9, 0.0)
    o.step()
    assert abs(p.values()[0] - 0.9) < 1e-5
    o.step()
    assert abs(p.values()[0] - 0.71) < 1e-5
    p = Tensor.new([10.0], True)
    p.set_gradient([0.0])
    optim.SGD([p], 0.1, 0.0, 0.1).step()
    assert abs(p.values()[0] - 9.9) < 1e-5


def test_adam_kats():  # adam.rs:8-62
    p = Tensor.new([1.0], True)
    p.set_gradient([1.0])
    o = optim.Adam([p], 0.1, 0.9, 0.999, 1e-8, 0.0)
    o.step()
    assert abs(p.values()[0] - 0.9) < 1e-5
    o.step()
    assert abs(p.values()[0] - 0.8) < 1e-4
    o2 = optim.Adam.default([Tensor.new([1.0], True)], 0.001)
    o2.zero_grad()
    assert abs(o2.learning_rate() - 0.001) < 1e-9


def test_linear_forward_kat():  # tests/nn_layers.rs:7-45
    lin = nn.Linear.with_weights(3, 2, [0.1, 0.2, 0.3, 0.4, 0.5, 0.6], [0.1, 0.2])
    out = lin.forward(Tensor.new([1, 2, 3, 4, 5, 6.0], True, shape=(2, 3))).values()
    assert out.shape == (2, 2)
    assert np.abs(out.ravel() - [1.5, 3.4, 3.3, 7.9]).max() < 1e-5


def test_linear_new_deterministic_init():  # nn.rs:67-96: sin(0.123 i) * sqrt(1/in)
    lin = nn.Linear(4, 3)
    w = lin.weight.values().ravel()
    ref = np.sin(np.arange(12, dtype=np.float32) * np.float32(0.123)) * np.sqrt(np.float32(0.25))
    assert np.abs(w - ref).max() < 1e-6
    assert (lin.bias.values() == 0).all()


def test_zero_grad_and_second_backward_accumulates():  # tensor.rs:120-142
    x = Tensor.new([1.0, 2.0], True)
    y = x.mul(x)
    y.backward()
    assert x.gradient().tolist() == [2.0, 4.0]
    y.backward()  # leaf grads accumulate across backward calls
    assert x.gradient().tolist() == [4.0, 8.0]
    x.zero_grad()
    assert x.gradient().tolist() == [0.0, 0.0]


# --- broadcasting, unbroadcast modes ------------------------------------------------

def test_bias_grad_correct_and_reference_modes(rng=np.random.default_rng(3)):
    X, b = rand(rng, (6, 4)), rand(rng, 4)
    for mode in ("correct", "reference"):
        nr.set_unbroadcast_mode(mode)
        try:
            x = Tensor.new(X, True)
            bb = Tensor.new(b, True)
            y = x.add(bb).relu().sum()
            y.backward()
            mask = (X + b > 0).astype(np.float32)
            if mode == "correct":
                want = mask.sum(0)
            else:  # backward.rs:12-39 + tensor.rs:120-132
                want = np.zeros(4, np.float32)
                want[0] = mask.sum()
            assert_close(bb.gradient(), want, what=mode)
            assert_close(x.gradient(), mask)
        finally:
            nr.set_unbroadcast_mode("correct")


@pytest.mark.parametrize("op", ["sub", "mul", "div"])
def test_broadcast_binary_grads(op):
    rng = np.random.default_rng(11)
    A = rand(rng, (5, 7))
    Bv = rng.uniform(0.5, 2.0, 7).astype(np.float32)
    a, b = Tensor.new(A, True), Tensor.new(Bv, True)
    getattr(a, op)(b).sum().backward()
    A64, B64 = A.astype(np.float64), Bv.astype(np.float64)
    if op == "sub":
        ga, gb = np.ones_like(A64), -np.ones((5, 7)).sum(0)
    elif op == "mul":
        ga, gb = np.broadcast_to(B64, (5, 7)), A64.sum(0)
    else:
        ga, gb = np.broadcast_to(1 / B64, (5, 7)), (-A64 / B64 ** 2).sum(0)
    assert_close(a.gradient(), ga, what=op + " a")
    assert_close(b.gradient(), gb, what=op + " b")


def test_unary_chain_matches_oracle():
    rng = np.random.default_rng(5)
    X = rng.uniform(0.2, 2.0, (8, 16)).astype(np.float32)
    x = Tensor.new(X, True)
    y = x.log().tanh().exp().sigmoid().sqrt().sin()
    y.backward()
    # oracle chain in the same node order, float32 forwards from numpy
    l1 = np.log(X); t2 = np.tanh(l1); e3 = np.exp(t2); s4 = O.sigmoid(e3); q5 = np.sqrt(s4)
    g = np.ones_like(X)
    g = O.sin_backward(g, q5)
    g = O.sqrt_backward(g, s4)
    g = O.sigmoid_backward(g, s4)
    g = O.exp_backward(g, e3)
    g = O.tanh_backward(g, t2)
    g = O.log_backward(g, X)
    assert_close(x.gradient(), g, abs_tol=1e-5, rel_tol=2e-4)


def test_layernorm_softmax_gelu_nodes():
    rng = np.random.default_rng(8)
    X = rand(rng, (32, 64))
    G = rng.uniform(0.5, 1.5, 64).astype(np.float32)
    Bt = rand(rng, 64)
    W = rand(rng, (64, 64), 0.1)
    x, gm, bt = Tensor.new(X, True), Tensor.new(G, True), Tensor.new(Bt, True)
    w = Tensor.new(W, False)
    y = x.layer_norm(gm, bt).gelu().matmul(w).softmax()
    up = rand(rng, (32, 64))
    loss = y.mul(Tensor.new(up, False)).sum()
    loss.backward()
    # oracle: same chain
    ln, _, _ = O.layernorm_fwd(X, G, Bt)
    ge = O.gelu(ln)
    z = O.matmul_f64(ge, W)
    s = O.softmax_rows(z)
    dz = O.softmax_backward(s, up, f64=True)
    dge, _ = O.matmul_backward(dz, ge, W, need_b=False, f64=True)
    dln = O.gelu_backward(dge, ln)
    dx, dg, db = O.layernorm_backward(dln, X, G)
    assert_close(x.gradient(), dx, abs_tol=2e-5, rel_tol=1e-3, what="dx")
    assert_close(gm.gradient(), dg, abs_tol=2e-5, rel_tol=1e-3, what="dgamma")
    assert_close(bt.gradient(), db, abs_tol=2e-5, rel_tol=1e-3, what="dbeta")


# --- C1: 2-layer MLP train step ------------------------------------------------------

def _c1_model(p):
    l1 = nn.Linear.with_weights(784, 128, p["W1"], p["b1"])
    l2 = nn.Linear.with_weights(128, 10, p["W2"], p["b2"])
    return nn.Sequential([l1, nn.ReLU(), l2]), l1, l2


@pytest.mark.parametrize("mode", ["correct", "reference"])
@pytest.mark.parametrize("labels_api", [False, True])
def test_c1_mlp_step_matches_oracle(mode, labels_api):
    p = make_c1(seed=1)
    nr.set_unbroadcast_mode(mode)
    try:
        model, l1, l2 = _c1_model(p)
        opt = optim.SGD.simple(model.parameters(), 0.01)
        x = Tensor.new(p["x"], False)
        logits = model.forward(x)
        if labels_api:
            loss = logits.cross_entropy_labels(p["labels"])
        else:
            onehot = np.eye(10, dtype=np.float32)[p["labels"]]
            loss = logits.cross_entropy_loss(Tensor.new(onehot, False))
        loss.backward()
        ref_loss, grads, new = mlp_step(p, 0.01, mode)
        assert abs(loss.item() - ref_loss) <= 1e-5 + 1e-4 * abs(ref_loss)
        assert_contraction(l1.weight.gradient(), grads["W1"], 64, what="dW1")
        assert_contraction(l2.weight.gradient(), grads["W2"], 64, what="dW2")
        assert_close(l1.bias.gradient(), grads["b1"], what="db1")
        assert_close(l2.bias.gradient(), grads["b2"], what="db2")
        opt.step()
        opt.zero_grad()
        assert_close(l1.weight.values(), new["W1"], abs_tol=1e-6, rel_tol=1e-5, what="W1'")
        assert_close(l2.weight.values(), new["W2"], abs_tol=1e-6, rel_tol=1e-5, what="W2'")
        assert_close(l1.bias.values(), new["b1"], abs_tol=1e-6, rel_tol=1e-5, what="b1'")
        assert_close(l2.bias.values(), new["b2"], abs_tol=1e-6, rel_tol=1e-5, what="b2'")
        assert (l1.weight.gradient() == 0).all()
    finally:
        nr.set_unbroadcast_mode("correct")


def test_c1_mlp_three_steps_track_oracle():
    p = make_c1(seed=2)
    model, l1, l2 = _c1_model(p)
    opt = optim.SGD.simple(model.parameters(), 0.01)
    x = Tensor.new(p["x"], False)
    onehot = Tensor.new(np.eye(10, dtype=np.float32)[p["labels"]], False)
    cur = dict(p)
    for step in range(3):
        loss = model.forward(x).cross_entropy_loss(onehot)
        loss.backward()
        opt.step()
        opt.zero_grad()
        ref_loss, _, cur = mlp_step(cur, 0.01)
        assert abs(loss.item() - ref_loss) <= 2e-5 + 1e-4 * abs(ref_loss), step
    assert_close(l1.weight.values(), cur["W1"], abs_tol=1e-6, rel_tol=1e-5)
    assert_close(l2.weight.values(), cur["W2"], abs_tol=1e-6, rel_tol=1e-5)


def test_argmax_evaluate_rule():
    # Trainer::evaluate (train.rs:209-228): max_by => last maximum on ties.
    c = nr.default_context()
    logits = np.array([[1, 3, 3, 0], [5, 5, 1, 0]], np.float32)
    idx = c.empty((2,), np.int32)
    c.argmax_rows(c.to_device(logits), idx, tie_last=True)
    assert idx.numpy().tolist() == [2, 1]


def test_fused_linear_equals_reference_node_sequence():
    # nn.Linear's fused node vs the reference's Transpose -> MatMul -> Add nodes.
    p = make_c1(seed=3)
    onehot = np.eye(10, dtype=np.float32)[p["labels"]]
    grads = []
    for fused in (True, False):
        model, l1, l2 = _c1_model(p)
        l1.fused = l2.fused = fused
        loss = model.forward(Tensor.new(p["x"], False)).cross_entropy_loss(
            Tensor.new(onehot, False))
        loss.backward()
        grads.append([t.gradient() for t in (l1.weight, l1.bias, l2.weight, l2.bias)]
                     + [loss.item()])
    for a, b in zip(*grads):
        assert_close(a, b, abs_tol=1e-7, rel_tol=1e-6)


@pytest.mark.parametrize("T", [64, 2048])
def test_sequential_linear_relu_node_equals_two_nodes(monkeypatch, T):
    # Sequential's Linear+ReLU node vs the Linear node and the ReLU node: the
    # same loss and parameter gradients, bit for bit (T = 64 takes the tiny
    # kernel's fused epilogue and masked loads, T = 2048 the separate passes).
    rng = np.random.default_rng(T)
    p = make_c1(seed=5)
    x = rng.standard_normal((T, 784)).astype(np.float32)
    onehot = np.eye(10, dtype=np.float32)[rng.integers(0, 10, T)]
    out = []
    for fuse in (True, False):
        monkeypatch.setattr(nn.Sequential, "fuse_relu", fuse)
        model, l1, l2 = _c1_model(p)
        loss = model.forward(Tensor.new(x, False)).cross_entropy_loss(Tensor.new(onehot, False))
        loss.backward()
        out.append([loss.values()] + [t.gradient() for t in (l1.weight, l1.bias, l2.weight,
                                                              l2.bias)])
    for a, b in zip(*out):
        assert np.array_equal(a, b)
