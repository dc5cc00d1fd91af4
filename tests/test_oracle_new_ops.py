"""Pins the float64 oracles of the ops numrs lacks (attention block, LSTM)
against torch float64 autograd on tiny shapes -- an independent library, CPU
only, no GPU involved."""
import numpy as np
import pytest

from oracle import transformer_oracle as TO

torch = pytest.importorskip("torch")


def test_transformer_block_oracle_matches_torch_autograd():
    w, x, t, dims = TO.make_c4(seed=9, B=2, S=5, D=8, H=2, F=12)
    B, S, H = dims
    loss, g, _ = TO.block(w, x, t, dims)

    tw = {k: torch.tensor(v, dtype=torch.float64, requires_grad=True) for k, v in w.items()}
    D = x.shape[1]
    extra = {n: torch.zeros(D, dtype=torch.float64, requires_grad=True)
             for n in ("bq", "bk", "bv", "bo", "c2")}
    extra["c1"] = torch.zeros(w["w1"].shape[0], dtype=torch.float64, requires_grad=True)
    gam = {n: torch.ones(D, dtype=torch.float64, requires_grad=True) for n in ("g1", "g2")}
    bet = {n: torch.zeros(D, dtype=torch.float64, requires_grad=True) for n in ("b1", "b2")}
    tx = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    tt = torch.tensor(t, dtype=torch.float64)
    F = torch.nn.functional
    ln1 = F.layer_norm(tx, (D,), gam["g1"], bet["b1"], eps=1e-5)
    q = ln1 @ tw["wq"].T + extra["bq"]
    k = ln1 @ tw["wk"].T + extra["bk"]
    v = ln1 @ tw["wv"].T + extra["bv"]

    def hd(a):
        return a.reshape(B, S, H, -1).transpose(1, 2)

    att = torch.softmax(hd(q) @ hd(k).transpose(-1, -2) / (D // H) ** 0.5, -1) @ hd(v)
    A = att.transpose(1, 2).reshape(B * S, D)
    r = tx + A @ tw["wo"].T + extra["bo"]
    ln2 = F.layer_norm(r, (D,), gam["g2"], bet["b2"], eps=1e-5)
    y = r + F.gelu(ln2 @ tw["w1"].T + extra["c1"]) @ tw["w2"].T + extra["c2"]
    tl = ((y - tt) ** 2).mean()
    tl.backward()

    assert abs(loss - tl.item()) < 1e-12
    for k_ in ("wq", "wk", "wv", "wo", "w1", "w2"):
        np.testing.assert_allclose(g[k_], tw[k_].grad.numpy(), rtol=1e-9, atol=1e-12, err_msg=k_)
    np.testing.assert_allclose(g["x"], tx.grad.numpy(), rtol=1e-9, atol=1e-12)
    for ours, theirs in (("ln1_gamma", gam["g1"]), ("ln1_beta", bet["b1"]),
                         ("ln2_gamma", gam["g2"]), ("ln2_beta", bet["b2"]),
                         ("bq", extra["bq"]), ("bo", extra["bo"]), ("c1", extra["c1"]),
                         ("c2", extra["c2"])):
        np.testing.assert_allclose(g[ours], theirs.grad.numpy(), rtol=1e-9, atol=1e-12,
                                   err_msg=ours)


def test_lstm_forecaster_oracle_matches_torch_autograd():
    from oracle import lstm_oracle as LO

    layers, hw, hb, x, target = LO.make_c5(seed=3, B=3, T=6, I=4, H=5, n_layers=2)
    loss, g, _ = LO.forecaster(layers, hw, hb, x, target)

    lstm = torch.nn.LSTM(4, 5, num_layers=2, batch_first=True).double()
    with torch.no_grad():
        for li, l in enumerate(layers):
            getattr(lstm, f"weight_ih_l{li}").copy_(torch.tensor(l["w_ih"], dtype=torch.float64))
            getattr(lstm, f"weight_hh_l{li}").copy_(torch.tensor(l["w_hh"], dtype=torch.float64))
            getattr(lstm, f"bias_ih_l{li}").copy_(torch.tensor(l["b"], dtype=torch.float64))
            getattr(lstm, f"bias_hh_l{li}").zero_()
    tx = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    thw = torch.tensor(hw, dtype=torch.float64, requires_grad=True)
    thb = torch.tensor(hb, dtype=torch.float64, requires_grad=True)
    out, _ = lstm(tx)
    y = out[:, -1] @ thw.T + thb
    tl = ((y - torch.tensor(target, dtype=torch.float64)) ** 2).mean()
    tl.backward()
    assert abs(loss - tl.item()) < 1e-12
    for li in range(2):
        np.testing.assert_allclose(g[f"w_ih{li}"], getattr(lstm, f"weight_ih_l{li}").grad.numpy(),
                                   rtol=1e-9, atol=1e-13)
        np.testing.assert_allclose(g[f"w_hh{li}"], getattr(lstm, f"weight_hh_l{li}").grad.numpy(),
                                   rtol=1e-9, atol=1e-13)
        np.testing.assert_allclose(g[f"b{li}"], getattr(lstm, f"bias_ih_l{li}").grad.numpy(),
                                   rtol=1e-9, atol=1e-13)
    np.testing.assert_allclose(g["head_w"], thw.grad.numpy(), rtol=1e-9, atol=1e-13)
    np.testing.assert_allclose(g["x"], tx.grad.numpy(), rtol=1e-9, atol=1e-13)
