"""GPU parity of the optimizers beyond SGD/Adam, Lookahead, L-BFGS and the LR
schedulers against the oracle (oracle/numrs_oracle.c).

Bars: every elementwise optimizer is bit-exact (parameters and state) over
several steps on ragged multi-tensor sets; LAMB's moments are bit-exact and
its parameters within 1e-5 relative (its layer norms are blocked sums, the
reference's are sequential f32 sums, so the trust ratio differs by the
sums' rounding); L-BFGS within 1e-4 relative (its dot products
are blocked sums feeding the two-loop scalars); the schedulers' learning
rates are bit-exact (the same host float arithmetic).
"""
import numpy as np
import pytest

import numrs_amd as nr
from numrs_amd import HipError, Tensor, optim
from numrs_amd import _lib as L
from oracle import oracle as O
from tests.conftest import assert_bits

pytestmark = pytest.mark.gpu

F = np.float32
SIZES = [4097, 1, 0, 256, 33]  # ragged, single, empty, aligned, odd

# kind -> (hyperparameters, oracle step(p, g, s1, s2, t), uses slot 2)
KINDS = {
    "adamw": (L.OPT_ADAMW, (0.01, 0.9, 0.999, 1e-8, 0.05),
              lambda p, g, a, b, t: O.adamw_step(p, g, a, b, t, 0.01, 0.9, 0.999, 1e-8, 0.05)),
    "rmsprop": (L.OPT_RMSPROP, (0.01, 0.99, 1e-8, 0.0, 0.0),
                lambda p, g, a, b, t: O.rmsprop_step(p, g, a, b, 0.01, 0.99, 1e-8, 0.0, 0.0)),
    "rmsprop_mom_wd": (L.OPT_RMSPROP, (0.01, 0.9, 1e-8, 0.02, 0.9),
                       lambda p, g, a, b, t: O.rmsprop_step(p, g, a, b, 0.01, 0.9, 1e-8, 0.02,
                                                            0.9)),
    "adagrad": (L.OPT_ADAGRAD, (0.05, 1e-10, 0.1),
                lambda p, g, a, b, t: O.adagrad_step(p, g, a, 0.05, 1e-10, 0.1)),
    "nadam": (L.OPT_NADAM, (0.002, 0.9, 0.999, 1e-8, 0.01),
              lambda p, g, a, b, t: O.nadam_step(p, g, a, b, t, 0.002, 0.9, 0.999, 1e-8, 0.01)),
    "radam": (L.OPT_RADAM, (0.01, 0.9, 0.999, 1e-8, 0.0),
              lambda p, g, a, b, t: O.radam_step(p, g, a, b, t, 0.01, 0.9, 0.999, 1e-8, 0.0)),
    "adadelta": (L.OPT_ADADELTA, (0.95, 1e-6, 0.01),
                 lambda p, g, a, b, t: O.adadelta_step(p, g, a, b, 0.95, 1e-6, 0.01)),
    "adabound": (L.OPT_ADABOUND, (0.001, 0.1, 0.9, 0.999, 1e-8, 0.02, 0.01),
                 lambda p, g, a, b, t: O.adabound_step(p, g, a, b, t, 0.001, 0.1, 0.9, 0.999,
                                                       1e-8, 0.02, 0.01)),
    "rprop": (L.OPT_RPROP, (0.01, 1.2, 0.5, 1e-6, 50.0),
              lambda p, g, a, b, t: O.rprop_step(p, g, a, b, 1.2, 0.5, 1e-6, 50.0)),
}


def _no_slot2(name):
    return name in ("rmsprop", "adagrad")


@pytest.mark.parametrize("name", list(KINDS))
def test_optimizer_kernel_bit_exact(hip_ctx, name):
    """Seven steps (RAdam crosses its rectification threshold at t = 6) on a
    ragged multi-tensor set, every step's gradient fresh; p and both state
    slots bit-exact against the oracle after each step."""
    print(f"[gpu] optimizer kernel {name}", flush=True)
    c = hip_ctx
    kind, hyper, ostep = KINDS[name]
    rng = np.random.default_rng(11)
    ps = [rng.standard_normal(n).astype(F) for n in SIZES]
    init1 = hyper[0] if name == "rprop" else 0.0
    s1 = [np.full(n, init1, F) for n in SIZES]
    s2 = [np.zeros(n, F) for n in SIZES]
    dp = [c.to_device(p) for p in ps]
    d1 = [c.to_device(x) for x in s1]
    d2 = None if _no_slot2(name) else [c.to_device(x) for x in s2]
    for t in range(1, 8):
        gs = [rng.standard_normal(n).astype(F) for n in SIZES]
        if name == "rprop" and t == 3:  # zero and negative-zero gradients: signum(+-0)
            gs[3][:4] = np.array([0.0, -0.0, 0.0, -0.0], F)
        dg = [c.to_device(g) for g in gs]
        c.optimizer_step(kind, dp, dg, d1, d2, hyper, t)
        for i in range(len(SIZES)):
            ostep(ps[i], gs[i], s1[i], s2[i], t)
        for i in range(len(SIZES)):
            assert_bits(dp[i].numpy(), ps[i], f"{name} p[{i}] t={t}")
            assert_bits(d1[i].numpy(), s1[i], f"{name} s1[{i}] t={t}")
            if d2 is not None:
                assert_bits(d2[i].numpy(), s2[i], f"{name} s2[{i}] t={t}")


@pytest.mark.parametrize("wd", [0.0, 0.01])
def test_lamb_kernel(hip_ctx, wd):
    print(f"[gpu] lamb wd={wd}", flush=True)
    c = hip_ctx
    rng = np.random.default_rng(12)
    sizes = [70000, 5, 1, 2048]
    ps = [rng.standard_normal(n).astype(F) for n in sizes]
    ms = [np.zeros(n, F) for n in sizes]
    vs = [np.zeros(n, F) for n in sizes]
    dp, dm, dv = ([c.to_device(x) for x in xs] for xs in (ps, ms, vs))
    hyper = (0.01, 0.9, 0.999, 1e-6, wd)
    for t in range(1, 5):
        gs = [rng.standard_normal(n).astype(F) for n in sizes]
        c.optimizer_step(L.OPT_LAMB, dp, [c.to_device(g) for g in gs], dm, dv, hyper, t)
        for i in range(len(sizes)):
            O.lamb_step(ps[i], gs[i], ms[i], vs[i], t, *hyper)
            got = dp[i].numpy()
            assert_bits(dm[i].numpy(), ms[i], f"lamb m[{i}]")
            assert_bits(dv[i].numpy(), vs[i], f"lamb v[{i}]")
            # The trust ratio's norms are blocked sums here and sequential f32
            # sums in the reference (relative error up to ~n*2^-24 for n terms),
            # so p = p - lr*ratio*u agrees to lr*|u|*(ratio error).
            np.testing.assert_allclose(got, ps[i], rtol=1e-5, atol=2e-6)
            ps[i] = got.copy()  # continue from the GPU state


def test_lookahead_and_dot_kernels(hip_ctx):
    c = hip_ctx
    rng = np.random.default_rng(13)
    fast = [rng.standard_normal(n).astype(F) for n in (1000, 3)]
    slow = [rng.standard_normal(n).astype(F) for n in (1000, 3)]
    df, ds = [c.to_device(x) for x in fast], [c.to_device(x) for x in slow]
    c.lookahead_update(df, ds, 0.5)
    for f, s in zip(fast, slow):
        O.lookahead_sync(f, s, 0.5)
    for i in range(2):
        assert_bits(df[i].numpy(), fast[i], "fast")
        assert_bits(ds[i].numpy(), slow[i], "slow")
    # dot: exact on integer-valued inputs, else within fp32 rounding of float64
    a = np.arange(1, 3001, dtype=F) % 7
    out = c.empty(1)
    c.dot(c.to_device(a), c.to_device(a), out)
    assert out.numpy()[0] == F(np.sum(a.astype(np.float64) ** 2))
    x, y = rng.standard_normal(100001).astype(F), rng.standard_normal(100001).astype(F)
    c.dot(c.to_device(x), c.to_device(y), out)
    assert abs(out.numpy()[0] - x.astype(np.float64) @ y) <= 1e-5 * np.abs(x * y).sum()


def test_optimizer_step_errors(hip_ctx):
    c = hip_ctx
    p = c.to_device(np.ones(4, F))
    with pytest.raises(HipError):
        c.optimizer_step(99, [p], [p], [p], [p], (0.1,), 1)
    with pytest.raises(HipError):  # wrong hyperparameter count
        c.optimizer_step(L.OPT_ADAMW, [p], [p], [p], [p], (0.1, 0.9), 1)
    with pytest.raises(HipError):  # t < 1 for an Adam-family kind
        c.optimizer_step(L.OPT_NADAM, [p], [p], [p], [p], (0.1, 0.9, 0.999, 1e-8, 0.0), 0)
    with pytest.raises(HipError):  # missing second slot
        c.optimizer_step(L.OPT_ADAMW, [p], [p], [p], None, (0.1, 0.9, 0.999, 1e-8, 0.0), 1)


# --- through the Tensor API -------------------------------------------------------------

ENGINE = {
    "AdamW": (lambda ps: optim.AdamW(ps, 0.01, weight_decay=0.05), "adamw"),
    "RMSprop": (lambda ps: optim.RMSprop(ps, 0.01, 0.9, 1e-8, 0.02, 0.9), "rmsprop_mom_wd"),
    "AdaGrad": (lambda ps: optim.AdaGrad(ps, 0.05, 1e-10, 0.1), "adagrad"),
    "NAdam": (lambda ps: optim.NAdam(ps, 0.002, weight_decay=0.01), "nadam"),
    "RAdam": (lambda ps: optim.RAdam(ps, 0.01), "radam"),
    "AdaDelta": (lambda ps: optim.AdaDelta(ps, 0.95, 1e-6, 0.01), "adadelta"),
    "AdaBound": (lambda ps: optim.AdaBound(ps, 0.001, 0.1, 0.9, 0.999, 1e-8, 0.02, 0.01),
                 "adabound"),
    "Rprop": (lambda ps: optim.Rprop(ps, 0.01, 1.2, 0.5, 1e-6, 50.0), "rprop"),
}


@pytest.mark.parametrize("name", list(ENGINE))
def test_engine_optimizer_matches_oracle(hip_ctx, name):
    """Optimizer objects over tensors whose gradients come from a backward
    pass (y = sum(w * x)): the step counter, state and zero_grad behave as the
    reference's."""
    print(f"[gpu] engine optimizer {name}", flush=True)
    nr.set_default_context(hip_ctx)
    make, key = ENGINE[name]
    _, _, ostep = KINDS[key]
    rng = np.random.default_rng(14)
    w0 = [rng.standard_normal(n).astype(F) for n in (300, 7)]
    ws = [Tensor.new(w, True) for w in w0]
    opt = make(ws)
    ref = [w.copy() for w in w0]
    init1 = 0.01 if name == "Rprop" else 0.0
    s1 = [np.full(w.size, init1, F) for w in w0]
    s2 = [np.zeros(w.size, F) for w in w0]
    for t in range(1, 7):
        xs = [rng.standard_normal(w.size).astype(F) for w in w0]
        loss = None
        for w, x in zip(ws, xs):
            term = w.mul(Tensor.new(x, False)).sum()
            loss = term if loss is None else loss.add(term)
        loss.backward()
        opt.step()
        opt.zero_grad()
        for i in range(len(w0)):
            ostep(ref[i], xs[i], s1[i], s2[i], t)  # d(sum w*x)/dw = x
            assert_bits(ws[i].values(), ref[i], f"{name} w[{i}] t={t}")


def test_engine_lamb_and_rates(hip_ctx):
    nr.set_default_context(hip_ctx)
    rng = np.random.default_rng(15)
    w0 = rng.standard_normal(500).astype(F)
    w = Tensor.new(w0, True)
    opt = optim.LAMB([w], 0.01)
    ref, m, v = w0.copy(), np.zeros(500, F), np.zeros(500, F)
    for t in range(1, 4):
        x = rng.standard_normal(500).astype(F)
        w.mul(Tensor.new(x, False)).sum().backward()
        opt.step()
        opt.zero_grad()
        O.lamb_step(ref, x, m, v, t, 0.01, 0.9, 0.999, 1e-6, 0.01)
        np.testing.assert_allclose(w.values(), ref, rtol=1e-5, atol=2e-6)
        ref = w.values().copy()
    # learning-rate accessors: AdaDelta reads 1 and ignores sets; Rprop is the
    # mean step size and a set resets every step size
    ad = optim.AdaDelta([Tensor.new(np.ones(3, F), True)])
    ad.set_learning_rate(0.5)
    assert ad.learning_rate() == 1.0
    rp = optim.Rprop([Tensor.new(np.ones(5, F), True), Tensor.new(np.ones(2, F), True)], 0.25)
    assert rp.learning_rate() == F(0.25)
    rp.set_learning_rate(0.125)
    assert rp.learning_rate() == F(0.125)
    aw = optim.AdamW.default([Tensor.new(np.ones(3, F), True)], 0.003)
    aw.set_learning_rate(0.004)
    assert aw.learning_rate() == F(0.004)


def test_engine_reference_kats(hip_ctx):
    """tests/autograd/optim/standard_opts.rs and advanced_opts.rs through the
    Tensor API (parameter 10 or 1, gradient set directly)."""
    nr.set_default_context(hip_ctx)

    def run(make, val, grad, steps=1):
        p = Tensor.new(np.array([val], F), True)
        opt = make([p])
        for gv in grad if isinstance(grad, list) else [grad] * steps:
            p.set_gradient(np.array([gv], F))
            opt.step()
        return float(p.values()[0])

    assert run(lambda ps: optim.AdamW(ps, 0.1, 0.9, 0.999, 1e-8, 0.1), 10.0, 0.0) < 10.0
    assert run(lambda ps: optim.AdaGrad(ps, 0.01, 1e-10, 0.1), 10.0, 1.0) < 10.0
    assert run(lambda ps: optim.AdaDelta(ps, 0.9, 1e-6, 0.0), 1.0, 1.0) != 1.0
    assert run(lambda ps: optim.NAdam(ps, 0.002, 0.9, 0.999, 1e-8, 0.0), 1.0, 1.0) < 1.0
    assert run(lambda ps: optim.RAdam(ps, 0.001, 0.9, 0.999, 1e-8, 0.0), 1.0, 1.0) < 1.0
    assert run(lambda ps: optim.LAMB(ps, 0.001, 0.9, 0.999, 1e-8, 0.0), 1.0, 1.0) < 1.0
    assert run(lambda ps: optim.Rprop(ps, 0.01, 0.5, 1.2, 1e-6, 50.0), 1.0, 1.0) < 1.0
    assert run(lambda ps: optim.Rprop(ps, 0.01, 0.5, 1.2, 1e-6, 50.0), 1.0, [1.0, -1.0]) != 1.0
    assert run(lambda ps: optim.AdaBound(ps, 0.01, 0.1, 0.9, 0.999, 1e-8, 0.0, 0.1), 0.0, 100.0,
               steps=5) < 0.0
    p1 = run(lambda ps: optim.RMSprop(ps, 0.01, 0.99, 1e-8, 0.0, 0.9), 1.0, 1.0, steps=1)
    p2 = run(lambda ps: optim.RMSprop(ps, 0.01, 0.99, 1e-8, 0.0, 0.9), 1.0, 1.0, steps=2)
    assert p2 < p1


def test_engine_lookahead(hip_ctx):
    """Lookahead(SGD, k=2, alpha=0.5): two inner steps, then the slow sync."""
    nr.set_default_context(hip_ctx)
    rng = np.random.default_rng(16)
    w0 = rng.standard_normal(64).astype(F)
    w = Tensor.new(w0, True)
    opt = optim.Lookahead(optim.SGD.simple([w], 0.1), [w], k=2, alpha=0.5)
    ref, slow = w0.copy(), w0.copy()
    for step in range(1, 6):
        x = rng.standard_normal(64).astype(F)
        w.mul(Tensor.new(x, False)).sum().backward()
        opt.step()
        opt.zero_grad()
        O.sgd_step(ref, x, None, 0.1)
        if step % 2 == 0:
            O.lookahead_sync(ref, slow, 0.5)
        assert_bits(w.values(), ref, f"lookahead step {step}")
    assert opt.learning_rate() == F(0.1)


def test_engine_lbfgs_quadratic(hip_ctx):
    """L-BFGS on f(w) = 0.5 w^T A w - b^T w (grads through the engine: A w via
    a matmul node) against the oracle's L-BFGS, and the loss decreases."""
    nr.set_default_context(hip_ctx)
    rng = np.random.default_rng(17)
    n = 16
    Q = rng.standard_normal((n, n)).astype(F)
    A = (Q @ Q.T / n + np.eye(n, dtype=F)).astype(F)
    b = rng.standard_normal(n).astype(F)
    w0 = rng.standard_normal(n).astype(F)
    w = Tensor.new(w0.reshape(n, 1), True)
    opt = optim.LBFGS([w], lr=0.3, history_size=4)
    ref = O.LBFGS(lr=0.3, history_size=4)
    x = [w0.copy()]
    At, bt = Tensor.new(A, False), Tensor.new(b.reshape(n, 1), False)
    for _ in range(6):
        # grad of 0.5 w^T A w - b^T w is A w - b: build it as d/dw of sum((0.5 A w - b) * w)
        aw = At.matmul(w)
        f = aw.mul(Tensor.new(np.full((n, 1), 0.5, F), False)).sub(bt).mul(w).sum()
        f.backward()
        g = w.gradient().ravel().copy()
        opt.step()
        opt.zero_grad()
        ref.step(x, [g])
        np.testing.assert_allclose(w.values().ravel(), x[0], rtol=1e-4, atol=1e-5)
        x[0] = w.values().ravel().copy()  # continue from the GPU iterate
    fv = lambda z: 0.5 * z @ A.astype(np.float64) @ z - b @ z  # noqa: E731
    assert fv(x[0].astype(np.float64)) < fv(w0.astype(np.float64))


@pytest.mark.parametrize("kind", ["step", "exponential", "cosine", "warmup", "plateau"])
def test_schedulers_match_oracle(hip_ctx, kind):
    nr.set_default_context(hip_ctx)
    w = Tensor.new(np.ones(3, F), True)
    opt = optim.SGD.simple([w], 0.1)
    args = {"step": (3, 0.5), "exponential": (0.9,), "cosine": (10, 0.001), "warmup": (4, 0.0),
            "plateau": (0.5, 2, 0.01)}[kind]
    sched = {"step": optim.StepLR, "exponential": optim.ExponentialLR,
             "cosine": optim.CosineAnnealingLR, "warmup": optim.LinearWarmup,
             "plateau": optim.ReduceLROnPlateau}[kind](*args)
    ref = O.Scheduler(kind, *args)
    lr = F(0.1)
    metrics = [1.0, 0.9, 0.95, 0.95, 0.8, 0.85, 0.9, 0.9, 0.9, 0.9, 0.9, 0.9]
    for e in range(12):
        if kind == "plateau":
            sched.step_with_metric(metrics[e], opt)
            lr = ref.step(lr, F(metrics[e]))
        else:
            sched.step(opt)
            lr = ref.step(lr)
        assert F(opt.learning_rate()) == lr, (kind, e)
    if kind == "plateau":
        with pytest.raises(RuntimeError):
            sched.step(opt)
