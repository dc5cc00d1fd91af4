"""Pins the oracle's restatements of the optimizers beyond SGD/Adam, the
Lookahead update, L-BFGS and the LR schedulers (CPU only).

What fixes each one:
  * the reference's own tests (numrs-core/tests/autograd/optim/
    standard_opts.rs, advanced_opts.rs), run through the oracle;
  * each update rule written again in float64 from the formulas in the
    reference's doc comments, over several steps on random data (a dropped
    term, a wrong sign or a swapped beta fails these);
  * special cases with known exact results: Rprop's sign logic and
    f32::signum(+0) = 1, RAdam's un-rectified branch, AdaBound's clipping,
    LAMB's trust ratio of 1 for a zero parameter, schedulers' closed forms.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O

F = np.float32


def rnd(rng, n, scale=1.0):
    return (rng.standard_normal(n) * scale).astype(np.float32)


def close(a, b, rtol=2e-5, atol=1e-6):
    np.testing.assert_allclose(np.asarray(a, np.float64), np.asarray(b, np.float64), rtol=rtol,
                               atol=atol)


# --- the reference's KATs (direction checks) -----------------------------------

def one(v):
    return np.array([v], np.float32)


def test_standard_opts_kats():
    # test_adamw_weight_decay: zero gradient, decay alone lowers p
    p, m, v = one(10.0), one(0.0), one(0.0)
    O.adamw_step(p, one(0.0), m, v, 1, 0.1, 0.9, 0.999, 1e-8, 0.1)
    assert p[0] < 10.0
    # test_rmsprop_momentum: second step moves further
    p, v, b = one(1.0), one(0.0), one(0.0)
    O.rmsprop_step(p, one(1.0), v, b, 0.01, 0.99, 1e-8, 0.0, 0.9)
    p1 = p[0]
    O.rmsprop_step(p, one(1.0), v, b, 0.01, 0.99, 1e-8, 0.0, 0.9)
    assert p[0] < p1
    # test_adagrad_weight_decay / basic
    p, a = one(10.0), one(0.0)
    O.adagrad_step(p, one(1.0), a, 0.01, 1e-10, 0.1)
    assert p[0] < 10.0
    p, a = one(1.0), one(0.0)
    O.adagrad_step(p, one(1.0), a, 0.01, 1e-10, 0.0)
    assert p[0] < 1.0
    # test_adamw_basic, test_rmsprop_basic
    p, m, v = one(1.0), one(0.0), one(0.0)
    O.adamw_step(p, one(1.0), m, v, 1, 0.1, 0.9, 0.999, 1e-8, 0.1)
    assert p[0] < 1.0
    p, v, b = one(1.0), one(0.0), one(0.0)
    O.rmsprop_step(p, one(1.0), v, b, 0.01, 0.99, 1e-8, 0.0, 0.0)
    assert p[0] < 1.0
    # test_adadelta_basic
    p, eg, ed = one(1.0), one(0.0), one(0.0)
    O.adadelta_step(p, one(1.0), eg, ed, 0.9, 1e-6, 0.0)
    assert p[0] != 1.0


def test_advanced_opts_kats():
    p, m, v = one(1.0), one(0.0), one(0.0)
    O.nadam_step(p, one(1.0), m, v, 1, 0.002, 0.9, 0.999, 1e-8, 0.0)
    assert p[0] < 1.0
    p, m, v = one(1.0), one(0.0), one(0.0)
    O.radam_step(p, one(1.0), m, v, 1, 0.001, 0.9, 0.999, 1e-8, 0.0)
    assert p[0] < 1.0
    p, m, v = one(1.0), one(0.0), one(0.0)
    O.lamb_step(p, one(1.0), m, v, 1, 0.001, 0.9, 0.999, 1e-8, 0.0)
    assert p[0] < 1.0
    # test_rprop_basic: Rprop::new(params, 0.01, 0.5, 1.2, 1e-6, 50.0)
    p, st, pv = one(1.0), one(0.01), one(0.0)
    O.rprop_step(p, one(1.0), st, pv, 0.5, 1.2, 1e-6, 50.0)
    assert p[0] < 1.0
    # test_adabound_basic
    p, m, v = one(1.0), one(0.0), one(0.0)
    O.adabound_step(p, one(1.0), m, v, 1, 0.001, 0.1, 0.9, 0.999, 1e-8, 0.0, 0.001)
    assert p[0] < 1.0
    # test_rprop_sign_flip: +1 then -1
    p, st, pv = one(1.0), one(0.01), one(0.0)
    O.rprop_step(p, one(1.0), st, pv, 0.5, 1.2, 1e-6, 50.0)
    O.rprop_step(p, one(-1.0), st, pv, 0.5, 1.2, 1e-6, 50.0)
    assert p[0] != 1.0
    # test_adabound_clipping: five steps from 0 with g = 100 move p below 0
    p, m, v = one(0.0), one(0.0), one(0.0)
    for t in range(1, 6):
        O.adabound_step(p, one(100.0), m, v, t, 0.01, 0.1, 0.9, 0.999, 1e-8, 0.0, 0.1)
    assert p[0] < 0.0


# --- float64 closed forms over several steps --------------------------------------

STEPS = 5


def _grads(rng, n):
    return [rnd(rng, n) for _ in range(STEPS)]


@pytest.mark.parametrize("wd", [0.0, 0.05])
def test_adamw_closed_form(wd):
    rng = np.random.default_rng(1)
    n, lr, b1, b2, eps = 257, 0.01, 0.9, 0.999, 1e-8
    p = rnd(rng, n)
    m, v = np.zeros(n, F), np.zeros(n, F)
    P, M, V = p.astype(np.float64), np.zeros(n), np.zeros(n)
    for t, g in enumerate(_grads(rng, n), 1):
        O.adamw_step(p, g, m, v, t, lr, b1, b2, eps, wd)
        M = b1 * M + (1 - b1) * g
        V = b2 * V + (1 - b2) * g.astype(np.float64) ** 2
        mh, vh = M / (1 - b1 ** t), V / (1 - b2 ** t)
        P = P - lr * (mh / (np.sqrt(vh) + eps) + wd * P)
    close(p, P, rtol=1e-5)
    close(m, M)
    close(v, V)


@pytest.mark.parametrize("wd,mom", [(0.0, 0.0), (0.01, 0.0), (0.0, 0.9), (0.02, 0.5)])
def test_rmsprop_closed_form(wd, mom):
    rng = np.random.default_rng(2)
    n, lr, alpha, eps = 300, 0.01, 0.99, 1e-8
    p = rnd(rng, n)
    v, b = np.zeros(n, F), np.zeros(n, F)
    P, Vv, B = p.astype(np.float64), np.zeros(n), np.zeros(n)
    for g in _grads(rng, n):
        O.rmsprop_step(p, g, v, b, lr, alpha, eps, wd, mom)
        G = g + wd * P
        Vv = alpha * Vv + (1 - alpha) * G * G
        if mom > 0:
            B = mom * B + G / (np.sqrt(Vv) + eps)
            P = P - lr * B
        else:
            P = P - lr * G / (np.sqrt(Vv) + eps)
    close(p, P, rtol=1e-5)
    close(v, Vv)


@pytest.mark.parametrize("wd", [0.0, 0.1])
def test_adagrad_closed_form(wd):
    rng = np.random.default_rng(3)
    n, lr, eps = 129, 0.05, 1e-10
    p = rnd(rng, n)
    acc = np.zeros(n, F)
    P, A = p.astype(np.float64), np.zeros(n)
    for g in _grads(rng, n):
        O.adagrad_step(p, g, acc, lr, eps, wd)
        G = g + wd * P
        A = A + G * G
        P = P - lr * G / (np.sqrt(A) + eps)
    close(p, P, rtol=1e-5)
    close(acc, A)


@pytest.mark.parametrize("wd", [0.0, 0.01])
def test_nadam_closed_form(wd):
    rng = np.random.default_rng(4)
    n, lr, b1, b2, eps = 200, 0.002, 0.9, 0.999, 1e-8
    p = rnd(rng, n)
    m, v = np.zeros(n, F), np.zeros(n, F)
    P, M, V = p.astype(np.float64), np.zeros(n), np.zeros(n)
    for t, g in enumerate(_grads(rng, n), 1):
        O.nadam_step(p, g, m, v, t, lr, b1, b2, eps, wd)
        G = g + wd * P
        M = b1 * M + (1 - b1) * G
        V = b2 * V + (1 - b2) * G * G
        bc1, bc2 = 1 - b1 ** t, 1 - b2 ** t
        mbar = b1 * (M / bc1) + (1 - b1) * G / bc1
        P = P - lr * mbar / (np.sqrt(V / bc2) + eps)
    close(p, P, rtol=1e-5)


def _radam64(P, g, M, V, t, lr, b1, b2, eps):
    M = b1 * M + (1 - b1) * g
    V = b2 * V + (1 - b2) * g * g
    bc1, bc2 = 1 - b1 ** t, 1 - b2 ** t
    rho_inf = 2 / (1 - b2) - 1
    rho_t = rho_inf - 2 * t * b2 ** t / bc2
    if rho_t > 5:
        r = math.sqrt((rho_t - 4) * (rho_t - 2) * rho_inf / ((rho_inf - 4) * (rho_inf - 2) * rho_t))
        P = P - lr * r * (M / bc1) / (np.sqrt(V / bc2) + eps)
    else:
        P = P - lr * (M / bc1)
    return P, M, V, rho_t > 5


def test_radam_closed_form_both_branches():
    rng = np.random.default_rng(5)
    n, lr, b1, b2, eps = 150, 0.01, 0.9, 0.999, 1e-8
    p = rnd(rng, n)
    m, v = np.zeros(n, F), np.zeros(n, F)
    P, M, V = p.astype(np.float64), np.zeros(n), np.zeros(n)
    seen = set()
    for t in range(1, 9):  # rho_t crosses 5 between t = 5 and t = 6 for b2 = 0.999
        g = rnd(rng, n)
        adaptive = O.radam_step(p, g, m, v, t, lr, b1, b2, eps, 0.0)
        P, M, V, a64 = _radam64(P, g.astype(np.float64), M, V, t, lr, b1, b2, eps)
        assert adaptive == a64
        seen.add(adaptive)
        close(p, P, rtol=1e-5)
    assert seen == {False, True}


def test_radam_unrectified_branch_is_bias_corrected_momentum():
    p, m, v = np.array([2.0, -1.0], F), np.zeros(2, F), np.zeros(2, F)
    g = np.array([0.5, 4.0], F)
    assert not O.radam_step(p, g, m, v, 1, 0.1, 0.9, 0.999, 1e-8, 0.0)
    # t = 1: m = 0.1 g, m_hat = m / 0.1 = g, p -= lr g
    close(p, np.array([2.0, -1.0]) - 0.1 * np.array([0.5, 4.0]), rtol=1e-6)


@pytest.mark.parametrize("wd", [0.0, 0.01])
def test_adadelta_closed_form(wd):
    rng = np.random.default_rng(6)
    n, rho, eps = 90, 0.95, 1e-6
    p = rnd(rng, n)
    eg, ed = np.zeros(n, F), np.zeros(n, F)
    P, EG, ED = p.astype(np.float64), np.zeros(n), np.zeros(n)
    for g in _grads(rng, n):
        O.adadelta_step(p, g, eg, ed, rho, eps, wd)
        G = g + wd * P
        EG = rho * EG + (1 - rho) * G * G
        D = np.sqrt(ED + eps) / np.sqrt(EG + eps) * G
        ED = rho * ED + (1 - rho) * D * D
        P = P - D
    close(p, P, rtol=1e-5)
    close(ed, ED, rtol=1e-5)


@pytest.mark.parametrize("wd", [0.0, 0.02])
def test_adabound_closed_form(wd):
    rng = np.random.default_rng(7)
    n, lr, flr, b1, b2, eps, gam = 120, 0.001, 0.1, 0.9, 0.999, 1e-8, 0.01
    p = rnd(rng, n)
    m, v = np.zeros(n, F), np.zeros(n, F)
    P, M, V = p.astype(np.float64), np.zeros(n), np.zeros(n)
    for t, g in enumerate(_grads(rng, n), 1):
        O.adabound_step(p, g, m, v, t, lr, flr, b1, b2, eps, wd, gam)
        G = g + wd * P
        M = b1 * M + (1 - b1) * G
        V = b2 * V + (1 - b2) * G * G
        bc1, bc2 = 1 - b1 ** t, 1 - b2 ** t
        lo, hi = flr * (1 - 1 / (gam * t + 1)), flr * (1 + 1 / (gam * t))
        step = lr * math.sqrt(bc2) / bc1
        lr_t = np.clip(step / (np.sqrt(V / bc2) + eps), lo, hi)
        P = P - lr_t * (M / bc1)
    close(p, P, rtol=1e-5)


def test_adabound_bounds_bind():
    # A huge first-step rate is clipped to the upper bound final_lr*(1+1/(gamma t)).
    p, m, v = one(0.0), one(0.0), one(0.0)
    O.adabound_step(p, one(1e-6), m, v, 1, 10.0, 0.1, 0.9, 0.999, 1e-8, 0.0, 0.5)
    hi = 0.1 * (1 + 1 / 0.5)
    close(p, [-hi * 1e-6], rtol=1e-5)


@pytest.mark.parametrize("wd", [0.0, 0.01])
def test_lamb_closed_form(wd):
    rng = np.random.default_rng(8)
    n, lr, b1, b2, eps = 333, 0.01, 0.9, 0.999, 1e-6
    p = rnd(rng, n)
    m, v = np.zeros(n, F), np.zeros(n, F)
    P, M, V = p.astype(np.float64), np.zeros(n), np.zeros(n)
    for t, g in enumerate(_grads(rng, n), 1):
        ratio = O.lamb_step(p, g, m, v, t, lr, b1, b2, eps, wd)
        M = b1 * M + (1 - b1) * g
        V = b2 * V + (1 - b2) * g.astype(np.float64) ** 2
        U = (M / (1 - b1 ** t)) / (np.sqrt(V / (1 - b2 ** t)) + eps)
        if wd > 0:
            U = U + wd * P
        r64 = np.linalg.norm(P) / np.linalg.norm(U)
        close(ratio, r64, rtol=1e-5)
        P = P - lr * r64 * U
    close(p, P, rtol=1e-5)


def test_lamb_trust_ratio_one_for_zero_weights():
    p, m, v = np.zeros(4, F), np.zeros(4, F), np.zeros(4, F)
    assert O.lamb_step(p, np.ones(4, F), m, v, 1, 0.1, 0.9, 0.999, 1e-6, 0.0) == 1.0


def test_rprop_sign_logic_exact():
    eta_p, eta_m, lo, hi = 1.2, 0.5, 1e-6, 50.0
    p = np.array([1.0, 1.0, 1.0, 1.0, 1.0], F)
    st = np.full(5, 0.25, F)
    pv = np.zeros(5, F)
    # first step: prev = 0 -> plain step of sign(g); signum(+0) = 1, signum(-0) = -1
    g1 = np.array([2.0, -3.0, 0.0, -0.0, 1.0], F)
    O.rprop_step(p, g1, st, pv, eta_p, eta_m, lo, hi)
    assert p.tolist() == [0.75, 1.25, 0.75, 1.25, 0.75]
    assert pv.tolist() == g1.tolist() and st.tolist() == [0.25] * 5
    # second step: same sign grows the step and moves; a flip shrinks it and holds
    g2 = np.array([1.0, 4.0, 5.0, 1.0, -2.0], F)
    O.rprop_step(p, g2, st, pv, eta_p, eta_m, lo, hi)
    assert st[0] == F(F(0.25) * F(eta_p)) and p[0] == F(F(0.75) - st[0])
    assert st[1] == F(F(0.25) * F(eta_m)) and p[1] == F(1.25) and pv[1] == 0.0
    assert st[4] == F(F(0.25) * F(eta_m)) and p[4] == F(0.75) and pv[4] == 0.0
    # prev was +-0 for elements 2 and 3: product 0 -> plain step again
    assert st[2] == F(0.25) and p[2] == F(F(0.75) - F(0.25)) and pv[2] == 5.0


def test_rprop_step_limits():
    p, st, pv = one(0.0), one(40.0), one(1.0)
    O.rprop_step(p, one(1.0), st, pv, 2.0, 0.5, 1e-3, 50.0)
    assert st[0] == 50.0  # min(80, lr_max)
    p, st, pv = one(0.0), one(2e-3), one(1.0)
    O.rprop_step(p, one(-1.0), st, pv, 2.0, 0.25, 1e-3, 50.0)
    assert st[0] == F(1e-3)  # max(5e-4, lr_min)


def test_lookahead_sync_closed_form():
    fast = np.array([1.0, 2.0, -4.0], F)
    slow = np.array([0.0, 2.0, 4.0], F)
    O.lookahead_sync(fast, slow, 0.5)
    assert slow.tolist() == [0.5, 2.0, 0.0] and fast.tolist() == slow.tolist()


def test_dot_seq_exact_on_integers():
    a = np.arange(1, 101, dtype=F)
    assert O.dot_seq(a, a) == F(sum(i * i for i in range(1, 101)))


# --- L-BFGS ------------------------------------------------------------------------

def _lbfgs64(x, grad, lr, hist, steps):
    """The same algorithm in float64 (lbfgs.rs:114-212)."""
    S, Y, px, pg = [], [], None, None
    for _ in range(steps):
        g = grad(x)
        if px is not None:
            s, y = x - px, g - pg
            if s @ y > 1e-10:
                S.append(s)
                Y.append(y)
                if len(S) > hist:
                    S.pop(0)
                    Y.pop(0)
        if not S:
            d = -g
        else:
            q = g.copy()
            al, rh = [0.0] * len(S), [0.0] * len(S)
            for i in reversed(range(len(S))):
                rh[i] = 1 / max(Y[i] @ S[i], 1e-10)
                al[i] = rh[i] * (S[i] @ q)
                q = q - al[i] * Y[i]
            r = (S[-1] @ Y[-1]) / max(Y[-1] @ Y[-1], 1e-10) * q
            for i in range(len(S)):
                b = rh[i] * (Y[i] @ r)
                r = r + S[i] * (al[i] - b)
            d = -r
        px, pg = x.copy(), g
        x = x + lr * d
    return x


def test_lbfgs_oracle_matches_float64_on_quadratic():
    rng = np.random.default_rng(9)
    n = 12
    Q = rng.standard_normal((n, n))
    A = (Q @ Q.T / n + np.eye(n)).astype(np.float64)
    b = rng.standard_normal(n)
    grad64 = lambda x: A @ x - b  # noqa: E731
    x0 = rng.standard_normal(n).astype(F)
    opt = O.LBFGS(lr=0.3, history_size=4)
    x = [x0.copy()]
    for _ in range(8):
        g = (A.astype(F) @ x[0] - b.astype(F)).astype(F)
        opt.step(x, [g])
    ref = _lbfgs64(x0.astype(np.float64), grad64, 0.3, 4, 8)
    close(x[0], ref, rtol=1e-3, atol=1e-4)
    # and it descends: the quadratic's value drops
    f = lambda z: 0.5 * z @ A @ z - b @ z  # noqa: E731
    assert f(x[0].astype(np.float64)) < f(x0.astype(np.float64))


# --- LR schedulers --------------------------------------------------------------------

def test_step_lr_closed_form():
    s, lr = O.Scheduler("step", 3, 0.5), F(0.1)
    trace = []
    for _ in range(10):
        lr = s.step(lr)
        trace.append(lr)
    want, cur = [], F(0.1)
    for e in range(1, 11):
        if e % 3 == 0:
            cur = F(cur * F(0.5))
        want.append(cur)
    assert trace == want


def test_exponential_lr_closed_form():
    s, lr = O.Scheduler("exponential", 0.9), F(1.0)
    for k in range(1, 6):
        lr = s.step(lr)
        close(lr, 0.9 ** k, rtol=1e-6)


def test_cosine_closed_form():
    s, lr = O.Scheduler("cosine", 10, 0.001), F(0.1)
    for t in range(1, 11):
        lr = s.step(lr)
        close(lr, 0.001 + (0.1 - 0.001) * (1 + math.cos(math.pi * t / 10)) / 2, rtol=1e-5,
              atol=1e-8)
    close(lr, 0.001, rtol=1e-5)


def test_warmup_closed_form():
    s, lr = O.Scheduler("warmup", 4, 0.0), F(0.2)
    trace = []
    for _ in range(6):
        lr = s.step(lr)
        trace.append(float(lr))
    close(trace, [0.05, 0.1, 0.15, 0.2, 0.2, 0.2], rtol=1e-6)


def test_plateau_trace():
    s, lr = O.Scheduler("plateau", 0.5, 2, 0.01), F(0.1)
    metrics = [1.0, 0.9, 0.95, 0.95, 0.8, 0.85, 0.9, 0.9, 0.9, 0.9, 0.9, 0.9]
    trace = []
    for mtr in metrics:
        lr = s.step(lr, F(mtr))
        trace.append(float(lr))
    # two epochs without improvement halve the lr (then the count restarts);
    # min_lr bounds it
    close(trace, [0.1, 0.1, 0.1, 0.05, 0.05, 0.05, 0.025, 0.025, 0.0125, 0.0125, 0.01, 0.01],
          rtol=1e-6)
