"""LSTM (N4) forward / BPTT and the C5 forecaster on the GPU against the
float64 oracle (tests/lstm_oracle.py, pinned to torch autograd)."""
import numpy as np
import pytest

import numrs_amd as nr
from numrs_amd import Tensor, nn
from tests import lstm_oracle as LO

pytestmark = pytest.mark.gpu


def _norm_rel(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)


@pytest.mark.parametrize("dims", [dict(B=3, T=6, I=4, H=5), dict(B=8, T=20, I=16, H=64),
                                  dict(B=5, T=9, I=70, H=130),
                                  dict(B=64, T=128, I=64, H=256),
                                  dict(B=3, T=4, I=8, H=1040), dict(B=2, T=3, I=8, H=2056)],
                         ids=["tiny", "medium", "ragged", "baseline",
                              "wide_unstaged_bwd", "wide_unstaged"])
def test_lstm_forecaster_matches_oracle(hip_ctx, dims):
    print(f"[gpu] lstm forecaster {dims}", flush=True)
    nr.set_default_context(hip_ctx)
    layers, hw, hb, x, target = LO.make_c5(seed=7, n_layers=2, **dims)
    model = nn.LSTMForecaster(layers, hw, hb)
    xt = Tensor.new(x, True)
    y = model.forward(xt)
    loss = y.mse_loss(Tensor.new(target, False))
    loss.backward()
    ref_loss, g, ref_y = LO.forecaster(layers, hw, hb, x, target)
    assert _norm_rel(y.values(), ref_y) < 1e-5
    assert abs(loss.item() - ref_loss) <= 1e-5 * abs(ref_loss) + 1e-7
    got = {"head_w": model.head.weight, "head_b": model.head.bias, "x": xt}
    for li, layer in enumerate(model.layers):
        got[f"w_ih{li}"], got[f"w_hh{li}"], got[f"b{li}"] = layer.w_ih, layer.w_hh, layer.bias
    for name, tensor in got.items():
        gg, rr = tensor.gradient(), g[name]
        # fp32 BPTT through 2 x T steps against float64: norm-wise relative error
        # and every element within 1e-3 of the tensor's largest gradient.
        assert _norm_rel(gg, rr) < 5e-4, (name, _norm_rel(gg, rr))
        assert np.abs(gg - rr).max() <= 1e-3 * np.abs(rr).max(), name


def test_time_slice_grad(hip_ctx):
    nr.set_default_context(hip_ctx)
    x = Tensor.new(np.arange(24, dtype=np.float32).reshape(2, 3, 4), True)
    y = x.time_slice(1)
    assert y.values().tolist() == [[4, 5, 6, 7], [16, 17, 18, 19]]
    y.sum().backward()
    g = x.gradient()
    assert (g[:, 1] == 1).all() and (g[:, 0] == 0).all() and (g[:, 2] == 0).all()
