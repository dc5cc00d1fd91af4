"""The HIP path against the committed golden fixtures (tests/golden/*.npz,
torch float64 autograd), through numrs's own tensor API: build the graph,
call backward(), read gradient(), exactly as the Rust tests drive Tensor.

An upstream grad G enters as loss = sum(out * G): mul_backward hands G to
the node under test unchanged (g * 1) and sum_backward seeds ones.
"""
from __future__ import annotations

import numpy as np
import pytest

import numrs_amd as nr
from numrs_amd import Tensor, nn, optim
from tests.conftest import assert_close
from tests.golden import fixtures

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def ctx(hip_ctx):
    nr.set_default_context(hip_ctx)
    nr.set_unbroadcast_mode("correct")
    yield hip_ctx


@pytest.fixture(scope="module")
def gs():
    return fixtures.grads_small()


def leaf(a):
    return Tensor.new(np.asarray(a, np.float32), True)


def const(a):
    return Tensor.new(np.asarray(a, np.float32), False)


def backprop(out, G):
    out.mul(const(G)).sum().backward()


def test_matmul(gs):
    a, b = leaf(gs["mm_A"]), leaf(gs["mm_B"])
    backprop(a.matmul(b), gs["mm_G"])
    assert_close(a.gradient(), gs["mm_dA"], what="dA")
    assert_close(b.gradient(), gs["mm_dB"], what="dB")


UNARY = {"relu": "un_x", "sigmoid": "un_x", "tanh": "un_x", "exp": "un_x", "log": "un_xp",
         "sqrt": "un_xp", "sin": "un_x", "cos": "un_x", "tan": "un_xt", "gelu": "un_x",
         "pow3": "un_x"}


@pytest.mark.parametrize("name", sorted(UNARY))
def test_unary(gs, name):
    x = leaf(gs[UNARY[name]])
    y = x.pow(3.0) if name == "pow3" else getattr(x, name)()
    assert_close(y.values(), gs[f"un_{name}_y"], what=f"{name} forward")
    backprop(y, gs["un_g"])
    dx = x.gradient()
    assert_close(dx, gs[f"un_{name}_dx"], what=name)
    if name == "relu":  # strict x > 0 at +0 and -0
        assert dx[0] == 0.0 and dx[1] == 0.0


@pytest.mark.parametrize("name", ["add", "sub", "mul", "div"])
def test_binary_broadcast_bias(gs, name):
    X, b = leaf(gs["bin_X"]), leaf(gs["bin_b"])
    backprop(getattr(X, name)(b), gs["bin_G"])
    assert_close(X.gradient(), gs[f"bin_{name}_dX"], what=f"{name} dX")
    assert_close(b.gradient(), gs[f"bin_{name}_db"], what=f"{name} db")


def test_sum_mean(gs):
    s = leaf(gs["red_S"])
    out = s.sum()
    assert_close(out.values(), [gs["red_sum"]], what="sum")
    out.backward()
    assert_close(s.gradient(), gs["red_sum_dS"], what="sum grad")
    m = leaf(gs["red_S"])
    out = m.mean()
    assert_close(out.values(), [gs["red_mean"]], what="mean")
    out.backward()
    assert_close(m.gradient(), gs["red_mean_dS"], what="mean grad")


def test_mse(gs):
    p = leaf(gs["mse_P"])
    loss = p.mse_loss(const(gs["mse_T"]))
    assert_close(loss.values(), [gs["mse_loss"]], what="mse loss")
    loss.backward()
    assert_close(p.gradient(), gs["mse_dP"], what="mse dP")


def test_cross_entropy_labels_and_onehot(gs):
    lab = gs["ce_labels"]
    for onehot in (False, True):
        z = leaf(gs["ce_logits"])
        if onehot:
            loss = z.cross_entropy_loss(const(np.eye(10, dtype=np.float32)[lab]))
        else:
            loss = z.cross_entropy_labels(lab)
        assert_close(loss.values(), [gs["ce_loss"]], what="ce loss")
        loss.backward()
        assert_close(z.gradient(), gs["ce_dlogits"], what=f"ce dlogits onehot={onehot}")


def test_softmax(gs):
    x = leaf(gs["sm_X"])
    y = x.softmax(1)
    assert_close(y.values(), gs["sm_y"], what="softmax")
    backprop(y, gs["sm_G"])
    assert_close(x.gradient(), gs["sm_dX"], what="softmax dX")


def test_layernorm(gs):
    x, g, b = leaf(gs["ln_X"]), leaf(gs["ln_gamma"]), leaf(gs["ln_beta"])
    y = x.layer_norm(g, b, 1e-5)
    assert_close(y.values(), gs["ln_y"], what="ln y")
    backprop(y, gs["ln_G"])
    assert_close(x.gradient(), gs["ln_dX"], what="ln dX")
    assert_close(g.gradient(), gs["ln_dgamma"], what="ln dgamma")
    assert_close(b.gradient(), gs["ln_dbeta"], what="ln dbeta")


def test_attention(gs):
    B, S, H, _ = (int(v) for v in gs["att_shape"])
    q, k, v = leaf(gs["att_q"]), leaf(gs["att_k"]), leaf(gs["att_v"])
    o = q.attention(k, v, B, S, H)
    assert_close(o.values(), gs["att_o"], what="attention out")
    backprop(o, gs["att_dO"])
    for t, key in ((q, "att_dq"), (k, "att_dk"), (v, "att_dv")):
        assert_close(t.gradient(), gs[key], what=key)


def test_lstm_layer(gs):
    x, wih, whh, b = (leaf(gs[n]) for n in ("lstm_x", "lstm_wih", "lstm_whh", "lstm_b"))
    h = x.lstm(wih, whh, b)
    assert_close(h.values(), gs["lstm_h"], what="lstm h")
    backprop(h, gs["lstm_G"])
    for t, key in ((x, "lstm_dx"), (wih, "lstm_dwih"), (whh, "lstm_dwhh"), (b, "lstm_db")):
        assert_close(t.gradient(), gs[key], what=key)


def test_argmax_ties(hip_ctx, gs):
    X = hip_ctx.to_device(gs["am_X"])
    for tie_last, key in ((False, "am_first"), (True, "am_last")):
        idx = hip_ctx.empty((X.shape[0],), np.int32)
        hip_ctx.argmax_rows(X, idx, tie_last=tie_last)
        assert (idx.numpy() == gs[key]).all(), key


def test_sgd_and_adam(gs):
    p = leaf(gs["opt_p0"])
    opt = optim.SGD([p], 0.1, 0.9, 0.01)
    for s in range(3):
        p.set_gradient(gs["opt_g"][s])
        opt.step()
        assert_close(p.values(), gs["opt_sgd"][s], what=f"sgd step {s + 1}")
    p = leaf(gs["opt_p0"])
    opt = optim.Adam([p], 0.01, 0.9, 0.999, 1e-8, 0.0)
    for s in range(3):
        p.set_gradient(gs["opt_g"][s])
        opt.step()
        assert_close(p.values(), gs["opt_adam"][s], what=f"adam step {s + 1}")


def test_mlp_c1_step():
    # Linear 784->128, ReLU, Linear 128->10, CE on labels
    z = fixtures.mlp_c1()
    l1 = nn.Linear.with_weights(784, 128, z["W1"], z["b1"])
    l2 = nn.Linear.with_weights(128, 10, z["W2"], z["b2"])
    model = nn.Sequential([l1, nn.ReLU(), l2])
    loss = model(Tensor.new(z["x"], False)).cross_entropy_labels(z["labels"])
    assert_close(loss.values(), [z["loss"]], what="loss")
    loss.backward()
    W1, b1, W2, b2 = model.parameters()
    dW1 = W1.gradient()
    assert_close(dW1[:16], z["dW1_rows16"], what="dW1 rows")
    assert_close(dW1.astype(np.float64).sum(0), z["dW1_colsum"], abs_tol=1e-4,
                 what="dW1 column sums")
    for t, key in ((b1, "db1"), (W2, "dW2"), (b2, "db2")):
        assert_close(t.gradient(), z[key], what=key)
