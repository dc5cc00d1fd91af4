"""Checkpoint and resume of device-resident training state, on the GPU.

A run saved with numrs's checkpoint format (ops/model.rs:544-588) after three
steps and restored into fresh tensors and a fresh optimizer must continue
bit for bit like the uninterrupted run: parameters, optimizer state slots and
the step counter all travel through the file."""
import numpy as np
import pytest

import numrs_amd as nr
from numrs_amd import Tensor, checkpoint, nn, optim

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def ctx(hip_ctx):
    nr.set_default_context(hip_ctx)
    yield hip_ctx


def _model(rng, zero=False):
    f = (lambda s: np.zeros(s, np.float32)) if zero else \
        (lambda s: (rng.standard_normal(s) * 0.3).astype(np.float32))
    l1 = nn.Linear.with_weights(12, 16, f((16, 12)), f(16))
    l2 = nn.Linear.with_weights(16, 5, f((5, 16)), f(5))
    named = {"l1.weight": l1.weight, "l1.bias": l1.bias, "l2.weight": l2.weight,
             "l2.bias": l2.bias}
    return nn.Sequential([l1, nn.Tanh(), l2]), named


def _step(model, opt, x, t):
    loss = model.forward(x).mse_loss(t)
    loss.backward()
    opt.step()
    opt.zero_grad()
    return loss.item()


OPTS = {
    "sgd_momentum": lambda ps: optim.SGD(ps, 0.05, momentum=0.9),
    "adam": lambda ps: optim.Adam(ps, 0.01),
    "rmsprop_momentum": lambda ps: optim.RMSprop(ps, 0.01, momentum=0.5),
    "rmsprop": lambda ps: optim.RMSprop(ps, 0.01),
    "adagrad": lambda ps: optim.AdaGrad(ps, 0.1),
}


@pytest.mark.parametrize("name", list(OPTS))
def test_resume_is_bit_exact(tmp_path, name):
    rng = np.random.default_rng(7)
    X = rng.standard_normal((8, 12)).astype(np.float32)
    Tt = rng.standard_normal((8, 5)).astype(np.float32)
    x, t = Tensor.new(X, False), Tensor.new(Tt, False)
    model, named = _model(rng)
    opt = OPTS[name](model.parameters())
    for _ in range(3):
        loss = _step(model, opt, x, t)
    path = str(tmp_path / f"{name}.json")
    checkpoint.save_checkpoint(path, named, opt, epoch=1, iteration=3, loss=loss, name=name)
    for _ in range(2):
        _step(model, opt, x, t)

    model2, named2 = _model(rng, zero=True)
    opt2 = OPTS[name](model2.parameters())
    ck = checkpoint.load_checkpoint(path)
    assert ck.iteration == 3 and ck.name == name
    checkpoint.restore(ck, named2, opt2)
    for _ in range(2):
        _step(model2, opt2, x, t)
    for k in named:
        a, b = named[k].values(), named2[k].values()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (name, k)


def test_refuses_optimizers_outside_the_format(tmp_path):
    rng = np.random.default_rng(8)
    model, named = _model(rng)
    with pytest.raises(ValueError):
        checkpoint.save_checkpoint(str(tmp_path / "x.json"), named,
                                   optim.AdamW(model.parameters(), 0.01))


def test_restore_checks_shapes(tmp_path):
    rng = np.random.default_rng(9)
    model, named = _model(rng)
    path = str(tmp_path / "p.json")
    checkpoint.save_checkpoint(path, named)
    bad = {"l1.weight": Tensor.new(np.zeros((3, 3), np.float32), True)}
    with pytest.raises(ValueError):
        checkpoint.restore(checkpoint.load_checkpoint(path), bad)
