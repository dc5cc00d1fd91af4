"""A training step recorded into a HIP graph (numrs_hip_graph_*, StepGraph)
and replayed: every replay equals the same step run eagerly, bit for bit
(same kernels, same arguments), with eager work and synchronisations of the
program's own between the replays.  Recording refuses what a replay could
not repeat faithfully, and a refused recording leaves the context usable."""
import numpy as np
import pytest

import numrs_amd as nr
from numrs_amd import HipError, StepGraph, Tensor, nn, optim
from oracle.mlp_oracle import make_c1

pytestmark = pytest.mark.gpu


def _mlp(p):
    l1 = nn.Linear.with_weights(784, 128, p["W1"], p["b1"])
    l2 = nn.Linear.with_weights(128, 10, p["W2"], p["b2"])
    return nn.Sequential([l1, nn.ReLU(), l2]), [l1.weight, l1.bias, l2.weight, l2.bias]


def _step(model, opt, x, onehot):
    def step():
        loss = model.forward(x).cross_entropy_loss(onehot)
        loss.backward()
        opt.step()
        opt.zero_grad()
        return loss
    return step


def _eager_work(rng):
    # unrelated eager work: allocations from the same block cache, a
    # backward sweep and a host read-back between two replays
    a0 = rng.standard_normal((33, 7)).astype(np.float32)
    a = Tensor.new(a0, True)
    a.mul(a).sum().backward()
    assert np.array_equal(a.gradient(), 2 * a0)


def test_c1_step_graph_replays_equal_eager_steps(hip_ctx):
    """C1 (64x784 -> 128 -> ReLU -> 10, softmax CE, SGD 0.01)."""
    print("[gpu] graph: C1 step replays vs eager steps", flush=True)
    nr.set_default_context(hip_ctx)
    p = make_c1(seed=5)
    rng = np.random.default_rng(5)
    eager, pe = _mlp(p)
    recorded, pr = _mlp(p)
    x = Tensor.new(p["x"], False)
    onehot = Tensor.new(np.eye(10, dtype=np.float32)[p["labels"]], False)
    se = _step(eager, optim.SGD.simple(eager.parameters(), 0.01), x, onehot)
    sr = _step(recorded, optim.SGD.simple(recorded.parameters(), 0.01), x, onehot)
    # one eager step each first: every buffer the step needs then exists
    assert se().item() == sr().item()
    g = StepGraph(hip_ctx, sr)
    try:
        # recording runs nothing: both models are still one step in
        for a, b in zip(pe, pr):
            assert np.array_equal(a.values(), b.values())
        for k in range(5):
            want = se().item()
            g.replay()
            _eager_work(rng)
            hip_ctx.sync()
            assert g.outputs.item() == want, k
            for i, (a, b) in enumerate(zip(pe, pr)):
                assert np.array_equal(a.values(), b.values()), (k, i)
        # two replays queued back to back, then one read
        for _ in range(2):
            se()
        g.replay()
        g.replay()
        for i, (a, b) in enumerate(zip(pe, pr)):
            assert np.array_equal(a.values(), b.values()), ("back to back", i)
    finally:
        g.close()
    # after close the model keeps training eagerly
    assert np.isfinite(sr().item())


def test_recording_refuses_step_count_optimizers(hip_ctx):
    print("[gpu] graph: Adam refused while recording", flush=True)
    nr.set_default_context(hip_ctx)
    w = Tensor.new(np.linspace(-1, 1, 64, dtype=np.float32).reshape(8, 8), True)
    opt = optim.Adam([w], 0.01)

    def step():
        loss = w.mul(w).sum()
        loss.backward()
        opt.step()
        opt.zero_grad()
        return loss

    step()
    with pytest.raises(HipError, match="host-side step count"):
        StepGraph(hip_ctx, step)
    # the context is out of recording mode: eager work and a new recording
    # work.  The aborted recording's calls never ran, so the gradient its
    # backward would have written is zeroed first.
    opt.zero_grad()
    before = w.values()
    step()
    assert not np.array_equal(before, w.values())
    sgd = optim.SGD.simple([w], 0.1)

    def sgd_step():
        loss = w.mul(w).sum()
        loss.backward()
        sgd.step()
        sgd.zero_grad()
        return loss

    sgd_step()
    g = StepGraph(hip_ctx, sgd_step)
    try:
        v0 = w.values().astype(np.float64)
        g.replay()
        hip_ctx.sync()
        # d/dw sum(w*w) = 2w, so one SGD step scales w by 1 - 0.2
        np.testing.assert_allclose(w.values(), v0 * 0.8, rtol=1e-6, atol=1e-7)
    finally:
        g.close()


def test_recording_refuses_host_transfers(hip_ctx):
    print("[gpu] graph: host upload refused while recording", flush=True)
    nr.set_default_context(hip_ctx)
    with pytest.raises(HipError):
        StepGraph(hip_ctx, lambda: Tensor.new(np.ones(5, np.float32), False))
    t = Tensor.new(np.arange(5, dtype=np.float32), True)
    t.sum().backward()
    assert t.gradient().tolist() == [1.0] * 5


def test_workspace_growth_between_replays_keeps_graph_valid(hip_ctx):
    """Eager work between replays that grows the context's workspace (a
    split-K matmul backward with a long inner dimension, then an explicit
    reserve) must not free the region the recorded kernels address: every
    replay still equals an eager step bit for bit."""
    print("[gpu] graph: workspace growth between C1 replays", flush=True)
    nr.set_default_context(hip_ctx)
    p = make_c1(seed=9)
    eager, pe = _mlp(p)
    recorded, pr = _mlp(p)
    x = Tensor.new(p["x"], False)
    onehot = Tensor.new(np.eye(10, dtype=np.float32)[p["labels"]], False)
    se = _step(eager, optim.SGD.simple(eager.parameters(), 0.01), x, onehot)
    sr = _step(recorded, optim.SGD.simple(recorded.parameters(), 0.01), x, onehot)
    assert se().item() == sr().item()
    g = StepGraph(hip_ctx, sr)
    rng = np.random.default_rng(9)
    M, K, N = 128, 1 << 16, 128
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    dC = rng.standard_normal((M, N)).astype(np.float32)
    dA_d, dB_d = hip_ctx.zeros((M, K)), hip_ctx.zeros((K, N))
    A_d, B_d, dC_d = hip_ctx.to_device(A), hip_ctx.to_device(B), hip_ctx.to_device(dC)
    try:
        for k in range(3):
            want = se().item()
            g.replay()
            # eager growth between replays: a long-K product (split-K
            # partials), then a reserve well beyond anything used so far
            hip_ctx.matmul_backward(dC_d, A_d, B_d, dA_d, dB_d)
            hip_ctx.reserve((64 << 20) * (k + 1))
            hip_ctx.sync()
            assert g.outputs.item() == want, k
            for i, (a, b) in enumerate(zip(pe, pr)):
                assert np.array_equal(a.values(), b.values()), (k, i)
        ref = (A.astype(np.float64).T @ dC.astype(np.float64))
        got = dB_d.numpy().astype(np.float64)
        assert np.max(np.abs(got - ref)) <= 1e-3 * np.max(np.abs(ref))
    finally:
        g.close()
    # with no graph left the retired regions are gone and work continues
    hip_ctx.reserve(1 << 20)
    assert np.isfinite(sr().item())


def test_graph_destroy_during_recording_is_deferred(hip_ctx):
    """numrs_hip_graph_destroy called while another recording is open is
    queued and runs when that recording ends; the first graph's replays
    before that still work and the new graph replays correctly."""
    print("[gpu] graph: destroy during a recording", flush=True)
    nr.set_default_context(hip_ctx)
    w = Tensor.new(np.linspace(-1, 1, 64, dtype=np.float32).reshape(8, 8), True)
    sgd = optim.SGD.simple([w], 0.1)

    def step():
        loss = w.mul(w).sum()
        loss.backward()
        sgd.step()
        sgd.zero_grad()
        return loss

    step()
    g1 = StepGraph(hip_ctx, step)
    closed = []

    def step_closing_g1():
        g1.close()  # queued: the recording is open
        closed.append(True)
        return step()

    g2 = StepGraph(hip_ctx, step_closing_g1)
    assert closed == [True]
    try:
        with pytest.raises(RuntimeError, match="closed"):
            g1.replay()
        v0 = w.values().astype(np.float64)
        g2.replay()
        hip_ctx.sync()
        np.testing.assert_allclose(w.values(), v0 * 0.8, rtol=1e-6, atol=1e-7)
    finally:
        g2.close()
