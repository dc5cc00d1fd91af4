"""The oracle against the committed golden fixtures (tests/golden/*.npz,
written by tests/golden/make_golden.py from torch float64 autograd).

CPU only.  The fp32-faithful oracle functions (the reference's own operation
order) must meet the north-star tolerance against the float64 fixtures; the
float64 oracles of the new ops must agree to float64 precision.  Shapes are
non-square throughout, so a transposed operand or a swapped index fails.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O
from oracle import lstm_oracle, mlp_oracle, transformer_oracle
from tests.conftest import assert_close
from tests.golden import fixtures


@pytest.fixture(scope="module")
def gs():
    return fixtures.grads_small()


def f32(a):
    return np.asarray(a, np.float32)


def test_matmul_backward(gs):
    # backward.rs:113-149; fixture A[6,5] B[5,7]
    dA, dB = O.matmul_backward(gs["mm_G"], gs["mm_A"], gs["mm_B"])
    assert_close(dA, gs["mm_dA"], what="dA")
    assert_close(dB, gs["mm_dB"], what="dB")


# name -> (oracle fn, input key, saved value handed to the backward)
UNARY = {
    "relu": (O.relu_backward, "un_x", "x"),        # backward.rs:152-163
    "sigmoid": (O.sigmoid_backward, "un_x", "y"),  # backward.rs:166-177
    "tanh": (O.tanh_backward, "un_x", "y"),        # backward.rs:503-517
    "exp": (O.exp_backward, "un_x", "y"),          # backward.rs:180-190
    "log": (O.log_backward, "un_xp", "x"),         # backward.rs:193-205
    "sqrt": (O.sqrt_backward, "un_xp", "x"),       # backward.rs:441-463
    "sin": (O.sin_backward, "un_x", "x"),
    "cos": (O.cos_backward, "un_x", "x"),
    "tan": (O.tan_backward, "un_xt", "y"),
    "gelu": (O.gelu_backward, "un_x", "x"),        # new op, exact erf form
}


@pytest.mark.parametrize("name", sorted(UNARY))
def test_unary_backward(gs, name):
    fn, xkey, saved = UNARY[name]
    v = gs[xkey] if saved == "x" else f32(gs[f"un_{name}_y"])
    assert_close(fn(gs["un_g"], v), gs[f"un_{name}_dx"], what=name)


def test_relu_mask_is_strict(gs):
    # x[0] = +0 and x[1] = -0: numrs's strict x > 0 gives grad 0 at both.
    dx = O.relu_backward(gs["un_g"], gs["un_x"])
    assert dx[0] == 0.0 and dx[1] == 0.0 and gs["un_relu_dx"][0] == 0.0


def test_pow_backward(gs):
    # backward.rs:407-438 with n = 3
    assert_close(O.pow_backward(gs["un_g"], gs["un_x"], 3.0), gs["un_pow3_dx"], what="pow3")


@pytest.mark.parametrize("name", ["add", "sub", "mul", "div"])
def test_binary_backward_broadcast_bias(gs, name):
    # backward.rs:43-109; the bias row is broadcast over 5 rows, its grad is
    # the column reduction (sum_to_shape CORRECT)
    X, b, G = gs["bin_X"], gs["bin_b"], gs["bin_G"]
    bb = np.broadcast_to(b, X.shape).copy()
    if name == "add":
        dX, dbf = G.copy(), G.copy()
    elif name == "sub":
        dX, dbf = G.copy(), O.sub_backward(G)[1]
    elif name == "mul":
        dX, dbf = O.mul_backward(G, X, bb)
    else:
        dX, dbf = O.div_backward(G, X, bb)
    assert_close(dX, gs[f"bin_{name}_dX"], what=f"{name} dX")
    assert_close(O.sum_to_shape(dbf, b.shape), gs[f"bin_{name}_db"], what=f"{name} db")


def test_sum_mean(gs):
    S = gs["red_S"]
    assert_close(O.sum_backward(1.0, S.shape), gs["red_sum_dS"], what="sum grad")
    assert_close(O.mean_backward(1.0, S.shape), gs["red_mean_dS"], what="mean grad")
    assert_close(O.mean_fwd(S), gs["red_mean"], what="mean")
    assert_close(O.sum_seq(S.ravel()), gs["red_sum"], what="sum")


def test_mse(gs):
    P, T = gs["mse_P"], gs["mse_T"]
    assert_close(O.mse_loss(P, T), gs["mse_loss"], what="mse loss")
    dp, _ = O.mse_backward(1.0, P, T)
    assert_close(dp, gs["mse_dP"], what="mse dP")


def test_cross_entropy(gs):
    Lg, lab = gs["ce_logits"], gs["ce_labels"]
    onehot = np.eye(Lg.shape[1], dtype=np.float32)[lab]
    assert_close(O.cross_entropy_loss(Lg, onehot), gs["ce_loss"], what="ce loss")
    assert_close(O.cross_entropy_backward(1.0, Lg, onehot), gs["ce_dlogits"], what="ce dlogits")


def test_softmax(gs):
    y = O.softmax_rows(gs["sm_X"])
    assert_close(y, gs["sm_y"], what="softmax")
    assert_close(O.softmax_backward(f32(gs["sm_y"]), gs["sm_G"]), gs["sm_dX"], what="softmax dX")


def test_layernorm(gs):
    y, _, _ = O.layernorm_fwd(gs["ln_X"], gs["ln_gamma"], gs["ln_beta"])
    assert_close(y, gs["ln_y"], what="ln y")
    dx, dg, db = O.layernorm_backward(gs["ln_G"], gs["ln_X"], gs["ln_gamma"])
    assert_close(dx, gs["ln_dX"], what="ln dX")
    assert_close(dg, gs["ln_dgamma"], what="ln dgamma")
    assert_close(db, gs["ln_dbeta"], what="ln dbeta")


def test_attention(gs):
    B, S, H, _ = (int(v) for v in gs["att_shape"])
    q, k, v = (gs[n].astype(np.float64) for n in ("att_q", "att_k", "att_v"))
    o, cache = transformer_oracle.attention_forward(q, k, v, B, S, H)
    np.testing.assert_allclose(o, gs["att_o"], rtol=1e-10, atol=1e-12)
    dq, dk, dv = transformer_oracle.attention_backward(gs["att_dO"].astype(np.float64), cache,
                                                       B, S, H)
    for got, key in ((dq, "att_dq"), (dk, "att_dk"), (dv, "att_dv")):
        np.testing.assert_allclose(got, gs[key], rtol=1e-10, atol=1e-12, err_msg=key)


def test_lstm_layer(gs):
    x, wih, whh, b = (gs[n].astype(np.float64) for n in ("lstm_x", "lstm_wih", "lstm_whh",
                                                         "lstm_b"))
    h, cache = lstm_oracle.lstm_layer(x, wih, whh, b)
    np.testing.assert_allclose(h, gs["lstm_h"], rtol=1e-10, atol=1e-12)
    dx, dwi, dwh, db = lstm_oracle.lstm_layer_backward(x, wih, whh, h, cache,
                                                       gs["lstm_G"].astype(np.float64))
    for got, key in ((dx, "lstm_dx"), (dwi, "lstm_dwih"), (dwh, "lstm_dwhh"), (db, "lstm_db")):
        np.testing.assert_allclose(got, gs[key], rtol=1e-10, atol=1e-12, err_msg=key)


def test_argmax_ties(gs):
    # ops::argmax keeps the first maximum (scalar.rs:517-528); Trainer::evaluate
    # keeps the last (max_by, train.rs:213-228); the fixture plants ties
    X = gs["am_X"]
    assert (O.argmax_rows(X) == gs["am_first"]).all()
    assert (O.argmax_rows(X, tie_last=True) == gs["am_last"]).all()
    assert (gs["am_first"] != gs["am_last"]).any(), "the fixture has ties"


def test_sgd_momentum_weight_decay(gs):
    p, v = gs["opt_p0"].copy(), np.zeros(7, np.float32)
    for s in range(3):
        O.sgd_step(p, gs["opt_g"][s], v, 0.1, mu=0.9, wd=0.01)
        assert_close(p, gs["opt_sgd"][s], what=f"sgd step {s + 1}")


def test_adam(gs):
    p, m, v = gs["opt_p0"].copy(), np.zeros(7, np.float32), np.zeros(7, np.float32)
    for s in range(3):
        O.adam_step(p, gs["opt_g"][s], m, v, s + 1, lr=0.01)
        assert_close(p, gs["opt_adam"][s], what=f"adam step {s + 1}")


def test_mlp_c1_step():
    # BASELINE configs[0] at full size: loss and every parameter grad
    z = fixtures.mlp_c1()
    loss, grads, _ = mlp_oracle.mlp_step(z)
    assert_close(loss, z["loss"], what="loss")
    assert_close(grads["W1"][:16], z["dW1_rows16"], what="dW1 rows")
    assert_close(grads["W1"].astype(np.float64).sum(0), z["dW1_colsum"], abs_tol=1e-4,
                 what="dW1 column sums")
    for k in ("b1", "W2", "b2"):
        assert_close(grads[k], z[f"d{k}"], what=f"d{k}")
