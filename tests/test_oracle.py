"""Pins the CPU oracle (oracle/numrs_oracle.c) before it is trusted as the checker.

Each restated function is checked against something that does not retype its
formula: the reference's own known-answer tests (file:line cited), closed
forms computed independently in float64 numpy, finite differences of an
independent float64 forward, or brute force.  Chosen so that a dropped term,
a wrong sign/index or a transposed operand fails.
"""
import math

import numpy as np
import pytest

from oracle import oracle as O
from tests.conftest import assert_close, rand


@pytest.fixture(scope="module")
def rng():
    return np.random.default_rng(1234)


# ---------------------------------------------------------------------------
# Reference known-answer tests
# ---------------------------------------------------------------------------

def test_kat_matmul_backward():
    # numrs-core/tests/autograd_matmul.rs:6-47: A=[[1,2],[3,4]], B=I, dC=ones.
    A = np.array([[1, 2], [3, 4]], np.float32)
    B = np.eye(2, dtype=np.float32)
    dA, dB = O.matmul_backward(np.ones((2, 2), np.float32), A, B)
    assert dA.ravel().tolist() == [1, 1, 1, 1]
    assert dB.ravel().tolist() == [4, 4, 6, 6]


def test_kat_relu_backward():
    # tests/autograd_activations.rs:5-24: x=[-1,0,1], seed ones -> [0, 0(strict), 1].
    dx = O.relu_backward(np.ones(3), np.array([-1.0, 0.0, 1.0]))
    assert dx.tolist() == [0.0, 0.0, 1.0]


def test_kat_sigmoid_forward():
    # tests/autograd_activations.rs:26-37
    y = O.sigmoid(np.array([0.0, 2.0, -2.0]))
    assert y[0] == 0.5 and abs(y[1] - 0.880797) < 1e-5 and abs(y[2] - 0.119202) < 1e-5


def test_kat_mse():
    # tests/autograd_loss.rs:5-37: pred [1,2,3], target [1,2,5]: loss 4/3, grad [0,0,-4/3].
    p = np.array([1, 2, 3], np.float32)
    t = np.array([1, 2, 5], np.float32)
    assert abs(O.mse_loss(p, t) - 1.3333333) < 1e-5
    dp, dt = O.mse_backward(1.0, p, t)
    assert dp[0] == 0.0 and abs(dp[2] + 1.333333) < 1e-5
    assert (dt == -dp).all()


def test_kat_cross_entropy():
    # tests/autograd_loss.rs:40-54: logits [2,-1], one-hot class 0: loss < 0.1.
    loss = O.cross_entropy_loss(np.array([[2.0, -1.0]]), np.array([[1.0, 0.0]]))
    assert loss < 0.1
    assert abs(loss - (-math.log(math.exp(2) / (math.exp(2) + math.exp(-1))))) < 1e-6


def test_kat_sum_mean():
    # tests/autograd_reduction.rs:6-40
    x = np.array([1, 2, 3, 4], np.float32)
    assert O.sum_avx2_order(x) == 10.0
    assert O.sum_backward(10.0 * 0 + 1.0, (2, 2)).ravel().tolist() == [1, 1, 1, 1]
    assert O.mean_fwd(x) == 2.5
    assert O.mean_backward(1.0, (4,)).tolist() == [0.25] * 4


def test_kat_add_mul_graph():
    # tests/autograd_basic.rs:45-100: z = x*y (+x): dx = y (+1), dy = x.
    dx, dy = O.mul_backward(np.ones(2), np.array([2, 3.0]), np.array([4, 5.0]))
    assert dx.tolist() == [4, 5] and dy.tolist() == [2, 3]
    # complex graph x=2, y=3: add node gives dx 1, mul node gives y=3; accumulated -> 4.
    gx = np.zeros(1, np.float32)
    O.accumulate(gx, np.ones(1))                                # add_backward, x branch
    O.accumulate(gx, O.mul_backward(np.ones(1), np.array([2.0]), np.array([3.0]))[0])
    assert gx[0] == 4.0


def test_kat_sgd():
    # tests/autograd/optim/sgd.rs:8-28: lr 0.1 -> [0.99, 1.98]
    p = np.array([1.0, 2.0], np.float32)
    O.sgd_step(p, np.array([0.1, 0.2]), None, 0.1)
    assert abs(p[0] - 0.99) < 1e-5 and abs(p[1] - 1.98) < 1e-5
    # sgd.rs:30-60: momentum 0.9, two steps -> 0.9, 0.71
    p = np.array([1.0], np.float32)
    v = np.zeros(1, np.float32)
    O.sgd_step(p, np.ones(1), v, 0.1, 0.9)
    assert abs(p[0] - 0.9) < 1e-5
    O.sgd_step(p, np.ones(1), v, 0.1, 0.9)
    assert abs(p[0] - 0.71) < 1e-5
    # sgd.rs:62-80: weight decay 0.1 on p=10, g=0 -> 9.9
    p = np.array([10.0], np.float32)
    O.sgd_step(p, np.zeros(1), None, 0.1, 0.0, 0.1)
    assert abs(p[0] - 9.9) < 1e-5


def test_kat_adam():
    # tests/autograd/optim/adam.rs:8-62: lr 0.1, g=1: p -> 0.9 -> 0.8
    p = np.array([1.0], np.float32)
    m = np.zeros(1, np.float32)
    v = np.zeros(1, np.float32)
    O.adam_step(p, np.ones(1), m, v, 1, lr=0.1)
    assert abs(p[0] - 0.9) < 1e-5
    O.adam_step(p, np.ones(1), m, v, 2, lr=0.1)
    assert abs(p[0] - 0.8) < 1e-4


def test_kat_argmax():
    # tests/ops_reduction_complex.rs:27-46 (axis 1 rows) and ops/reduction/argmax.rs:49-98
    assert O.argmax_rows(np.array([[1, 5, 2], [9, 3, 4]], np.float32)).tolist() == [1, 0]
    assert O.argmax_rows(np.array([[1, 5, 2, 9, 3]], np.float32)).tolist() == [3]
    assert O.argmax_rows(np.array([[3, 1, 4, 1, 5]], np.float32)).tolist() == [4]
    assert O.argmax_rows(np.array([[10, 2, 3, 4]], np.float32)).tolist() == [0]
    assert O.argmax_rows(np.array([[1, 3, 2, 3, 1]], np.float32)).tolist() == [1]  # first tie
    assert O.argmax_rows(np.array([[-5, -2, -3, -4]], np.float32)).tolist() == [1]
    # Trainer::evaluate (train.rs:213-228) uses max_by: last of equal maxima.
    assert O.argmax_rows(np.array([[1, 3, 2, 3, 1]], np.float32), tie_last=True).tolist() == [3]


def test_kat_linear_forward():
    # tests/nn_layers.rs:7-45: x[2,3] @ W^T + b = [[1.5,3.4],[3.3,7.9]]
    x = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    W = np.array([[0.1, 0.2, 0.3], [0.4, 0.5, 0.6]], np.float32)
    y = O.matmul_f64(x, O.transpose(W)) + np.array([0.1, 0.2], np.float32)
    assert np.abs(y - np.array([[1.5, 3.4], [3.3, 7.9]])).max() < 1e-5


# ---------------------------------------------------------------------------
# Closed forms and brute force
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("M,K,N", [(5, 3, 7), (1, 9, 4), (33, 17, 29)])
def test_matmul_backward_closed_form(rng, M, K, N):
    A, B, dC = rand(rng, (M, K)), rand(rng, (K, N)), rand(rng, (M, N))
    rA = dC.astype(np.float64) @ B.astype(np.float64).T
    rB = A.astype(np.float64).T @ dC.astype(np.float64)
    for f64 in (False, True):
        dA, dB = O.matmul_backward(dC, A, B, f64=f64)
        assert_close(dA, rA, what=f"dA f64={f64}")
        assert_close(dB, rB, what=f"dB f64={f64}")


def test_reference_fp32_needs_contraction_allowance():
    """numrs's own fp32 loop misses the bare 1e-5 + 1e-4|r| bound against the
    exact (float64) gradient at K = 2048 on some elements, but stays inside the
    contraction allowance used for the GPU GEMM tests."""
    from tests.conftest import contraction_allowance

    rng = np.random.default_rng(5)
    M = K = N = 2048
    A = rng.standard_normal((M, K), dtype=np.float32)
    B = rng.standard_normal((K, N), dtype=np.float32)
    dC = rng.standard_normal((M, N), dtype=np.float32)
    a32, _ = O.matmul_backward(dC, A, B, need_b=False, rows_a=(0, 8))
    a64, _ = O.matmul_backward(dC, A, B, need_b=False, rows_a=(0, 8), f64=True)
    err = np.abs(a32[:8].astype(np.float64) - a64[:8])
    bare = 1e-5 + 1e-4 * np.abs(a64[:8].astype(np.float64))
    assert (err > bare).sum() > 0
    assert (err <= bare + contraction_allowance(N)).all()


def test_matmul_backward_row_ranges(rng):
    A, B, dC = rand(rng, (6, 4)), rand(rng, (4, 5)), rand(rng, (6, 5))
    full_a, full_b = O.matmul_backward(dC, A, B, f64=True)
    dA, dB = O.matmul_backward(dC, A, B, f64=True, rows_a=(2, 4), rows_b=(1, 3))
    assert np.array_equal(dA[2:4], full_a[2:4]) and np.isnan(dA[:2]).all()
    assert np.array_equal(dB[1:3], full_b[1:3]) and np.isnan(dB[3:]).all()


def test_softmax_backward_jacobian(rng):
    x = rand(rng, (6, 11), 2.0)
    y = O.softmax_rows(x).astype(np.float64)
    g = rand(rng, (6, 11))
    ref = np.stack([(np.diag(s) - np.outer(s, s)).T @ gg for s, gg in zip(y, g.astype(np.float64))])
    assert_close(O.softmax_backward(y.astype(np.float32), g), ref, what="softmax faithful")
    assert_close(O.softmax_backward(y.astype(np.float32), g, f64=True), ref, what="softmax f64")


def test_sum_orders_exact(rng):
    for n in (1, 7, 8, 13, 37, 1000):
        x = rng.integers(-50, 50, n).astype(np.float32)
        exact = float(x.astype(np.int64).sum())
        assert O.sum_avx2_order(x) == exact
        assert O.sum_seq(x) == exact


def test_threaded_sum_exact_and_single_thread_order(rng):
    # Integer-valued inputs sum exactly in any order: every chunking must give
    # the exact sum; one thread is the 8-lane order itself, bit for bit.
    for n in (0, 1, 7, 8, 13, 37, 1000, 100003):
        x = rng.integers(-50, 50, n).astype(np.float32)
        exact = float(x.astype(np.int64).sum())
        for t in (1, 2, 3, 8, 16):
            assert O.sum_avx2_order_mt(x, t) == exact, (n, t)
    y = rng.standard_normal(1 << 16).astype(np.float32)
    assert O.sum_avx2_order_mt(y, 1) == O.sum_avx2_order(y)
    # A dropped chunk fails: the sum of the halves.
    h = y.size // 2
    assert O.sum_avx2_order_mt(y, 2) == np.float32(O.sum_avx2_order(y[:h]) + O.sum_avx2_order(y[h:]))


def test_sum_to_shape_matches_numpy(rng):
    cases = [((4, 5), (5,)), ((4, 5), (1, 5)), ((4, 5), (4, 1)), ((3, 4, 5), (4, 1)),
             ((3, 4, 5), (3, 1, 5)), ((2, 3), (1,)), ((7,), (1,)), ((2, 3, 4), (2, 3, 4))]
    for gs, os_ in cases:
        g = rand(rng, gs)
        nd = len(gs)
        o = (1,) * (nd - len(os_)) + tuple(os_)
        axes = tuple(d for d in range(nd) if o[d] == 1 and gs[d] != 1)
        ref = g.astype(np.float64).sum(axis=axes, keepdims=True).reshape(os_)
        assert_close(O.sum_to_shape(g, os_), ref, what=f"{gs}->{os_}")


def test_unbroadcast_reference_is_element0_full_sum():
    # backward.rs:12-39 sums any mismatched grad to [1]; tensor.rs:120-132 zips it
    # into element 0 of the [out] bias grad: Linear bias grad = [sum dY, 0, 0...].
    g = np.arange(6, dtype=np.float32).reshape(2, 3)
    db = np.zeros(3, np.float32)
    O.unbroadcast_reference_accumulate(g, db)
    assert db.tolist() == [15.0, 0.0, 0.0]


def test_accumulate_zip_truncates():
    dst = np.ones(3, np.float32)
    O.accumulate(dst, np.array([5.0], np.float32))
    assert dst.tolist() == [6.0, 1.0, 1.0]


def test_powi_is_square_and_multiply():
    f = np.float32
    assert O.powi(0.9, 1) == f(0.9)
    assert O.powi(0.999, 2) == f(0.999) * f(0.999)
    # 3 = 0b11: r = a, a2 = a*a, r = a*a2
    a = f(0.999)
    assert O.powi(0.999, 3) == a * (a * a)
    # 5 = 0b101: r = a; a2 = a*a; a4 = a2*a2; r = a*a4
    assert O.powi(0.999, 5) == a * ((a * a) * (a * a))
    for t in range(1, 40):
        assert abs(float(O.powi(0.999, t)) - 0.999 ** t) < 1e-5


# ---------------------------------------------------------------------------
# Finite differences against independent float64 forwards
# ---------------------------------------------------------------------------

def _fd(f, x, h=1e-5):
    x = x.astype(np.float64)
    d = np.empty_like(x)
    for i in range(x.size):
        xp, xm = x.copy(), x.copy()
        xp.flat[i] += h
        xm.flat[i] -= h
        d.flat[i] = (f(xp) - f(xm)) / (2 * h)
    return d


def _sig(x):
    return 1 / (1 + np.exp(-x))


UNARY = [
    ("sigmoid", lambda x: _sig(x), lambda g, x: O.sigmoid_backward(g, _sig(x)), (-4, 4)),
    ("tanh", np.tanh, lambda g, x: O.tanh_backward(g, np.tanh(x)), (-3, 3)),
    ("exp", np.exp, lambda g, x: O.exp_backward(g, np.exp(x)), (-2, 2)),
    ("log", np.log, lambda g, x: O.log_backward(g, x), (0.2, 3)),
    ("sqrt", np.sqrt, lambda g, x: O.sqrt_backward(g, x), (0.2, 3)),
    ("sin", np.sin, lambda g, x: O.sin_backward(g, x), (-3, 3)),
    ("cos", np.cos, lambda g, x: O.cos_backward(g, x), (-3, 3)),
    ("tan", np.tan, lambda g, x: O.tan_backward(g, np.tan(x)), (-1.2, 1.2)),
    ("pow3", lambda x: x ** 3, lambda g, x: O.pow_backward(g, x, 3.0), (0.2, 2)),
    ("gelu", lambda x: x * 0.5 * (1 + np.vectorize(math.erf)(x / math.sqrt(2))),
     lambda g, x: O.gelu_backward(g, x), (-4, 4)),
]


@pytest.mark.parametrize("name,fwd,bwd,rng_", UNARY, ids=[u[0] for u in UNARY])
def test_unary_backward_finite_difference(rng, name, fwd, bwd, rng_):
    x = rng.uniform(*rng_, 40).astype(np.float32)
    g = rand(rng, 40)
    # elementwise derivative: d/dx_i sum_j g_j f(x_j) = g_i f'(x_i)
    ref = _fd(lambda v: (g.astype(np.float64) * fwd(v)).sum(), x)
    assert_close(bwd(g, x.astype(np.float32)), ref, abs_tol=2e-4, rel_tol=2e-3, what=name)


def test_relu_backward_finite_difference(rng):
    x = rng.uniform(-3, 3, 50).astype(np.float32)
    x[np.abs(x) < 1e-2] = 0.5
    g = rand(rng, 50)
    ref = _fd(lambda v: (g.astype(np.float64) * np.maximum(v, 0)).sum(), x)
    assert_close(O.relu_backward(g, x), ref, abs_tol=1e-4, rel_tol=1e-3)


def test_div_sub_backward_finite_difference(rng):
    x = rng.uniform(-2, 2, 20).astype(np.float32)
    y = rng.uniform(0.5, 2, 20).astype(np.float32) * rng.choice([-1, 1], 20).astype(np.float32)
    g = rand(rng, 20)
    g64 = g.astype(np.float64)
    dx, dy = O.div_backward(g, x, y)
    assert_close(dx, _fd(lambda v: (g64 * v / y).sum(), x), abs_tol=1e-4, rel_tol=1e-3)
    assert_close(dy, _fd(lambda v: (g64 * x / v).sum(), y), abs_tol=1e-4, rel_tol=1e-3)
    sx, sy = O.sub_backward(g)
    assert_close(sx, _fd(lambda v: (g64 * (v - y)).sum(), x), abs_tol=1e-4, rel_tol=1e-3)
    assert_close(sy, _fd(lambda v: (g64 * (x - v)).sum(), y), abs_tol=1e-4, rel_tol=1e-3)


def test_mse_backward_finite_difference(rng):
    p, t = rand(rng, 12), rand(rng, 12)
    dp, dt = O.mse_backward(1.0, p, t)
    assert_close(dp, _fd(lambda v: ((v - t) ** 2).mean(), p), abs_tol=1e-4, rel_tol=1e-3)
    assert_close(dt, _fd(lambda v: ((p - v) ** 2).mean(), t), abs_tol=1e-4, rel_tol=1e-3)


def test_cross_entropy_backward_finite_difference(rng):
    B, C = 5, 7
    x = rand(rng, (B, C), 2.0)
    t = np.eye(C, dtype=np.float32)[rng.integers(0, C, B)]

    def loss(v):
        v = v.reshape(B, C)
        m = v.max(1, keepdims=True)
        ls = v - m - np.log(np.exp(v - m).sum(1, keepdims=True))
        return -(t * ls).sum() / B

    ref = _fd(loss, x)
    assert_close(O.cross_entropy_backward(1.0, x, t), ref, abs_tol=1e-4, rel_tol=1e-3)
    assert abs(O.cross_entropy_loss(x, t) - loss(x.astype(np.float64))) < 1e-5


def test_layernorm_backward_finite_difference(rng):
    R, C = 3, 8
    x, g = rand(rng, (R, C)), rand(rng, (R, C))
    gamma = rng.uniform(0.5, 1.5, C).astype(np.float32)
    beta = rand(rng, C)
    eps = 1e-5
    g64 = g.astype(np.float64)

    def fwd(xv, gm, bt):
        mu = xv.mean(1, keepdims=True)
        var = ((xv - mu) ** 2).mean(1, keepdims=True)
        return (xv - mu) / np.sqrt(var + eps) * gm + bt

    dx, dgam, dbet = O.layernorm_backward(g, x, gamma, eps)
    x64, gm64, bt64 = x.astype(np.float64), gamma.astype(np.float64), beta.astype(np.float64)
    assert_close(dx, _fd(lambda v: (g64 * fwd(v.reshape(R, C), gm64, bt64)).sum(), x),
                 abs_tol=2e-4, rel_tol=2e-3, what="dx")
    assert_close(dgam, _fd(lambda v: (g64 * fwd(x64, v, bt64)).sum(), gamma),
                 abs_tol=2e-4, rel_tol=2e-3, what="dgamma")
    assert_close(dbet, _fd(lambda v: (g64 * fwd(x64, gm64, v)).sum(), beta),
                 abs_tol=2e-4, rel_tol=2e-3, what="dbeta")
    y, mean, rstd = O.layernorm_fwd(x, gamma, beta, eps)
    assert_close(y, fwd(x64, gm64, bt64), what="ln fwd")


# --- reshape / flatten (a22) ---------------------------------------------------

def test_kat_reshape_shapes():
    # ops/shape/reshape.rs:115-195
    assert O.reshape_shape(6, [3, 2]) == (3, 2)                     # test_reshape_basic
    assert O.reshape_shape(8, [2, 2, 2]) == (2, 2, 2)               # test_reshape_3d
    assert O.reshape_shape(6, [-1, 3]) == (2, 3)                    # test_reshape_infer_dimension
    assert O.reshape_shape(4, [-1, 2]) == (2, 2)                    # ..._infer_first_dimension
    assert O.reshape_shape(4, [-1]) == (4,)                         # test_reshape_flatten
    with pytest.raises(ValueError):
        O.reshape_shape(4, [2, 3])                                  # test_reshape_invalid_size
    with pytest.raises(ValueError):
        O.reshape_shape(4, [-1, -1])                                # test_reshape_multiple_infer
    assert O.reshape_shape(1, [1, 1, 1]) == (1, 1, 1)               # test_reshape_to_scalar_like
    assert O.reshape_shape(4, [2, 2]) == (2, 2)                     # test_reshape_identity
    with pytest.raises(ValueError):
        O.reshape_shape(0, [0, -1])     # "Cannot infer dimension when other dimensions are zero"
    with pytest.raises(ValueError):
        O.reshape_shape(6, [-2, 3])     # "Invalid dimension size"


def test_flatten_shapes():
    # ops/shape/flatten.rs:13-43: merge start..=end, end clamped to the last dim
    assert O.flatten_shape((2, 3, 4), 1, 2) == (2, 12)
    assert O.flatten_shape((2, 3, 4), 0, 1) == (6, 4)
    assert O.flatten_shape((2, 3, 4), 0, 99) == (24,)
    assert O.flatten_shape((2, 3, 4), 1, 1) == (2, 3, 4)
    with pytest.raises(ValueError):
        O.flatten_shape((2, 3, 4), 2, 1)


def test_reshape_backward_is_the_row_major_inverse(rng):
    # backward.rs:315-330: the grad keeps row-major order.  Reshaping forward
    # and then backward is the identity, and an index permutation of the
    # grad (a transposed operand) is caught on non-square shapes.
    g = rand(rng, (3, 8))
    dx = O.reshape_backward(g, (4, 6))
    assert dx.shape == (4, 6)
    assert np.array_equal(dx.ravel(), g.ravel())
    assert np.array_equal(O.reshape_backward(dx, (3, 8)), g)
    assert not np.array_equal(dx, g.T.reshape(4, 6))
    dx[0, 0] += 1.0                                 # a copy, not a view
    assert dx.ravel()[0] != g.ravel()[0]
