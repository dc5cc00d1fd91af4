"""GPU parity: every HIP kernel against the CPU oracle on identical seeded inputs.

Bars (north star): bit-exact for select/multiply/divide/sqrt kernels, the
optimizers and every integer path; |g - r| <= 1e-5 + 1e-4|r| against the
float64-accumulated oracle for reductions, whose summation order differs from
the reference's.  Matmul gradients (length-K fp32 contractions) add the fp32
rounding allowance 4*2^-24*K that numrs's own fp32 loop also needs, and must
be on average at least as close to the exact gradient as that loop is
(tests/conftest.py::assert_contraction).  At the full BASELINE matmul sizes
every output element is compared with a float64 host product, the fp32 loop
runs on sampled rows for the aggregate bar, and size-independent identities
(checksums of checksums, exact power-of-two linearity) are checked besides.
"""
import sys

import ctypes
import math

import numpy as np
import pytest

from numrs_amd import HipError
from numrs_amd import _lib as L
from oracle import oracle as O
from tests.conftest import (assert_bits, assert_close, assert_contraction, assert_sum, rand,
                            seq_colsum32)

pytestmark = pytest.mark.gpu


def say(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def rng():
    return np.random.default_rng(20261201)


# ---------------------------------------------------------------------------
# matmul_backward (backward.rs:113-149)
# ---------------------------------------------------------------------------

SMALL_GEMMS = [(1, 1, 1), (2, 2, 2), (5, 3, 7), (64, 784, 128), (64, 128, 10), (130, 70, 257),
               (128, 128, 128), (256, 96, 192), (33, 1, 65), (1, 300, 1), (300, 4, 260)]


@pytest.mark.parametrize("M,K,N", SMALL_GEMMS)
def test_matmul_backward_small(hip_ctx, rng, M, K, N):
    say(f"matmul_backward M={M} K={K} N={N}")
    A, B, dC = rand(rng, (M, K)), rand(rng, (K, N)), rand(rng, (M, N))
    dA_ref, dB_ref = O.matmul_backward(dC, A, B, f64=True)
    dA_32, dB_32 = O.matmul_backward(dC, A, B)  # numrs's own fp32 loops
    c = hip_ctx
    dA, dB = c.empty((M, K)), c.empty((K, N))
    c.matmul_backward(c.to_device(dC), c.to_device(A), c.to_device(B), dA, dB)
    assert_contraction(dA.numpy(), dA_ref, N, ref32=dA_32, what="dA")
    assert_contraction(dB.numpy(), dB_ref, M, ref32=dB_32, what="dB")


def test_matmul_backward_kat(hip_ctx):
    # numrs-core/tests/autograd_matmul.rs:6-47
    c = hip_ctx
    A = c.to_device(np.array([[1, 2], [3, 4]], np.float32))
    B = c.to_device(np.eye(2, dtype=np.float32))
    dC = c.to_device(np.ones((2, 2), np.float32))
    dA, dB = c.empty((2, 2)), c.empty((2, 2))
    c.matmul_backward(dC, A, B, dA, dB)
    assert dA.numpy().ravel().tolist() == [1, 1, 1, 1]
    assert dB.numpy().ravel().tolist() == [4, 4, 6, 6]


def test_matmul_backward_accumulate_and_skip(hip_ctx, rng):
    M, K, N = 96, 160, 72
    say("matmul_backward accumulate/skip")
    A, B, dC = rand(rng, (M, K)), rand(rng, (K, N)), rand(rng, (M, N))
    ga, gb = rand(rng, (M, K)), rand(rng, (K, N))
    dA_ref, dB_ref = O.matmul_backward(dC, A, B, f64=True)
    c = hip_ctx
    dA, dB = c.to_device(ga), c.to_device(gb)
    dCd, Ad, Bd = c.to_device(dC), c.to_device(A), c.to_device(B)
    c.matmul_backward(dCd, Ad, Bd, dA, dB, accumulate=True)
    assert_contraction(dA.numpy(), ga.astype(np.float64) + dA_ref, N, what="dA acc")
    assert_contraction(dB.numpy(), gb.astype(np.float64) + dB_ref, M, what="dB acc")
    only_b = c.to_device(np.full((K, N), 7.0, np.float32))
    c.matmul_backward(dCd, Ad, None, None, only_b)
    assert_contraction(only_b.numpy(), dB_ref, M, what="dB only")
    only_a = c.empty((M, K))
    c.matmul_backward(dCd, None, Bd, only_a, None)
    assert_contraction(only_a.numpy(), dA_ref, N, what="dA only")


def _checksums(dC, A, B):
    """sum(dA) and sum(dB) from O(n^2) float64 identities:
    sum_ij (dC B^T)_ij = sum_l (sum_i dC_il)(sum_j B_jl);
    sum_ij (A^T dC)_ij = sum_l (sum_i A_li)(sum_j dC_lj)."""
    d = dC.astype(np.float64)
    sa = float(d.sum(0) @ B.astype(np.float64).sum(0))
    sb = float(A.astype(np.float64).sum(1) @ d.sum(1))
    return sa, sb


@pytest.mark.parametrize("M,K,N", [(2048, 2048, 2048), (4096, 1024, 4096)])
def test_matmul_backward_baseline_sizes(hip_ctx, rng, M, K, N):
    say(f"matmul_backward baseline M={M} K={K} N={N}")
    A, B, dC = rand(rng, (M, K)), rand(rng, (K, N)), rand(rng, (M, N))
    c = hip_ctx
    dCd, Ad, Bd = c.to_device(dC), c.to_device(A), c.to_device(B)
    dA, dB = c.empty((M, K)), c.empty((K, N))
    c.matmul_backward(dCd, Ad, Bd, dA, dB)
    ga, gb = dA.numpy(), dB.numpy()
    # Every element of dA and dB against float64 host products (BLAS in
    # float64: exact to ~1e-13 here), under the per-element contraction bar.
    d64 = dC.astype(np.float64)
    ra = d64 @ B.astype(np.float64).T
    assert_contraction(ga, ra, N, what="dA (every element)")
    rb = A.astype(np.float64).T @ d64
    assert_contraction(gb, rb, M, what="dB (every element)")
    # The oracle's float64-accumulated rows (rounded once to fp32) agree with
    # the host product on sampled rows, and numrs's own fp32 loops
    # (backward.rs:123-146) on those rows give the aggregate bar: the GPU
    # result is on average closer to the exact gradient.
    def rounded_once(o, r):
        return (np.abs(o - r) <= 2.0 ** -23 * np.abs(r) + 1e-30).all()

    for r0 in (0, 127, 128, 1023, M - 2):
        rows = (r0, r0 + 2)
        o64, _ = O.matmul_backward(dC, A, B, need_b=False, f64=True, rows_a=rows)
        assert rounded_once(o64[r0:r0 + 2], ra[r0:r0 + 2]), f"oracle dA rows {r0}"
        r32, _ = O.matmul_backward(dC, A, B, need_b=False, rows_a=rows)
        assert_contraction(ga[r0:r0 + 2], ra[r0:r0 + 2], N, ref32=r32[r0:r0 + 2],
                           what=f"dA rows {r0}")
    for r0 in (0, 129, K // 2, K - 2):
        rows = (r0, r0 + 2)
        _, o64 = O.matmul_backward(dC, A, B, need_a=False, f64=True, rows_b=rows)
        assert rounded_once(o64[r0:r0 + 2], rb[r0:r0 + 2]), f"oracle dB rows {r0}"
        _, r32 = O.matmul_backward(dC, A, B, need_a=False, rows_b=rows)
        assert_contraction(gb[r0:r0 + 2], rb[r0:r0 + 2], M, ref32=r32[r0:r0 + 2],
                           what=f"dB rows {r0}")
    del ra, rb, d64
    # Whole-output identities.
    sa, sb = _checksums(dC, A, B)
    assert abs(ga.astype(np.float64).sum() - sa) <= 1e-4 * np.abs(ga).sum()
    assert abs(gb.astype(np.float64).sum() - sb) <= 1e-4 * np.abs(gb).sum()
    # Exact power-of-two linearity: dC*2 doubles every bit pattern's value.
    dC2 = c.to_device(dC * 2)
    dA2, dB2 = c.empty((M, K)), c.empty((K, N))
    c.matmul_backward(dC2, Ad, Bd, dA2, dB2)
    assert_bits(dA2.numpy(), ga * 2, "dA linearity")
    assert_bits(dB2.numpy(), gb * 2, "dB linearity")


# Streamed large-tile path (256 x 128 workgroup tiles, DMA ring): taken for
# aligned products with at least one such tile per CU.  Batches of 256 x 128
# products reach the 256-tile threshold at small sizes; reductions of 1..7
# and 32 tiles cover every prologue/tail case of the three-stage ring.
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("K", [32, 64, 96, 128, 160, 192, 224, 1024])
def test_matmul_streamed_batched(hip_ctx, rng, ta, tb, K):
    batch, M, N = 128, 256, 256
    say(f"streamed matmul batch={batch} M={M} K={K} N={N} ta={ta} tb={tb}")
    A = rand(rng, (batch, K, M) if ta else (batch, M, K))
    B = rand(rng, (batch, N, K) if tb else (batch, K, N))
    C0 = rand(rng, (batch, M, N))
    c = hip_ctx
    Ad, Bd = c.to_device(A), c.to_device(B)
    C = c.to_device(C0)
    c.matmul_batched(Ad, Bd, C, trans_a=bool(ta), trans_b=bool(tb), accumulate=True)
    a64 = A.astype(np.float64).transpose(0, 2, 1) if ta else A.astype(np.float64)
    b64 = B.astype(np.float64).transpose(0, 2, 1) if tb else B.astype(np.float64)
    ref = C0.astype(np.float64) + a64 @ b64
    assert_contraction(C.numpy(), ref, K, what="streamed C += A B")


# Batched products with [256, 64] outputs per batch (attention's per-head
# shape at C4): the planner takes the 64 x 64 mini tile, three workgroups per
# CU; reductions of 1, 3 and 8 tiles cover the ring's prologue cases.
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("K", [32, 96, 256])
def test_matmul_streamed_batched_mini(hip_ctx, rng, ta, tb, K):
    batch, M, N = 128, 256, 64
    say(f"streamed mini matmul batch={batch} M={M} K={K} N={N} ta={ta} tb={tb}")
    A = rand(rng, (batch, K, M) if ta else (batch, M, K))
    B = rand(rng, (batch, N, K) if tb else (batch, K, N))
    C0 = rand(rng, (batch, M, N))
    c = hip_ctx
    Ad, Bd = c.to_device(A), c.to_device(B)
    C = c.to_device(C0)
    c.matmul_batched(Ad, Bd, C, trans_a=bool(ta), trans_b=bool(tb), accumulate=True)
    a64 = A.astype(np.float64).transpose(0, 2, 1) if ta else A.astype(np.float64)
    b64 = B.astype(np.float64).transpose(0, 2, 1) if tb else B.astype(np.float64)
    ref = C0.astype(np.float64) + a64 @ b64
    assert_contraction(C.numpy(), ref, K, what="mini C += A B")
    # the matmul_backward pair at the same per-batch shape (dA NT + dB TN)
    dC = rand(rng, (batch, M, N))
    A2, B2 = rand(rng, (batch, M, K)), rand(rng, (batch, K, N))
    dA, dB = c.empty((batch, M, K)), c.empty((batch, K, N))
    c.matmul_backward_batched(c.to_device(dC), c.to_device(A2), c.to_device(B2), dA, dB)
    d64 = dC.astype(np.float64)
    assert_contraction(dA.numpy(), d64 @ B2.astype(np.float64).transpose(0, 2, 1), N, what="dA")
    assert_contraction(dB.numpy(), A2.astype(np.float64).transpose(0, 2, 1) @ d64, M, what="dB")


@pytest.mark.parametrize("acc", [False, True])
def test_matmul_backward_streamed(hip_ctx, rng, acc):
    """matmul_backward through the streamed pair kernel (dA NT + dB TN tiles
    in one grid) at a batched shape whose tile count reaches the threshold."""
    batch, M, K, N = 4, 2048, 1024, 256
    say(f"streamed matmul_backward batch={batch} M={M} K={K} N={N} acc={acc}")
    A, B, dC = rand(rng, (batch, M, K)), rand(rng, (batch, K, N)), rand(rng, (batch, M, N))
    ga0 = rand(rng, (batch, M, K)) if acc else np.zeros((batch, M, K), np.float32)
    gb0 = rand(rng, (batch, K, N)) if acc else np.zeros((batch, K, N), np.float32)
    c = hip_ctx
    dA, dB = c.to_device(ga0), c.to_device(gb0)
    c.matmul_backward_batched(c.to_device(dC), c.to_device(A), c.to_device(B), dA, dB,
                              accumulate=acc)
    d64 = dC.astype(np.float64)
    ra = ga0 + d64 @ B.astype(np.float64).transpose(0, 2, 1)
    rb = gb0 + A.astype(np.float64).transpose(0, 2, 1) @ d64
    assert_contraction(dA.numpy(), ra, N, what="dA")
    assert_contraction(dB.numpy(), rb, M, what="dB")


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,K,N", [(64, 784, 128), (37, 19, 53), (256, 256, 256)])
def test_matmul_forward(hip_ctx, rng, ta, tb, M, K, N):
    say(f"matmul ta={ta} tb={tb} {M}x{K}x{N}")
    A = rand(rng, (K, M) if ta else (M, K))
    B = rand(rng, (N, K) if tb else (K, N))
    ref = (A.T if ta else A).astype(np.float64) @ (B.T if tb else B).astype(np.float64)
    c = hip_ctx
    C = c.empty((M, N))
    c.matmul(c.to_device(A), c.to_device(B), C, trans_a=bool(ta), trans_b=bool(tb))
    assert_contraction(C.numpy(), ref, K)


# (32, 256, 128, 256): 256 tiles of 128 x 64 over the batch -- the batched
# small-tile streamed pair.
@pytest.mark.parametrize("bt,M,K,N", [(6, 40, 64, 72), (32, 256, 128, 256)])
def test_matmul_backward_batched(hip_ctx, rng, bt, M, K, N):
    say(f"matmul_backward_batched bt={bt} M={M} K={K} N={N}")
    A, B, dC = rand(rng, (bt, M, K)), rand(rng, (bt, K, N)), rand(rng, (bt, M, N))
    c = hip_ctx
    dA, dB = c.empty((bt, M, K)), c.empty((bt, K, N))
    c.matmul_backward_batched(c.to_device(dC), c.to_device(A), c.to_device(B), dA, dB)
    ga, gb = dA.numpy(), dB.numpy()
    for i in range(bt):
        ra, rb = O.matmul_backward(dC[i], A[i], B[i], f64=True)
        assert_contraction(ga[i], ra, N, what=f"dA[{i}]")
        assert_contraction(gb[i], rb, M, what=f"dB[{i}]")


def test_matmul_empty_reduction(hip_ctx):
    c = hip_ctx
    dC = c.zeros((3, 0))
    A = c.to_device(np.ones((3, 4), np.float32))
    B = c.zeros((4, 0))
    dA = c.to_device(np.full((3, 4), 5.0, np.float32))
    c.matmul_backward(dC, A, B, dA, None)
    assert (dA.numpy() == 0).all()


# ---------------------------------------------------------------------------
# Broadcast-reduce: relu + bias (C3), sum_to_shape
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 5), (64, 128), (65, 257), (200, 1000),
                                       (1030, 1540), (4099, 513), (4096, 4096)])
def test_relu_bias_backward(hip_ctx, rng, rows, cols):
    say(f"relu_bias_backward {rows}x{cols}")
    g, z = rand(rng, (rows, cols)), rand(rng, (rows, cols))
    z[0, 0] = 0.0  # strict '>' at zero
    c = hip_ctx
    gd, zd = c.to_device(g), c.to_device(z)
    dx, db = c.empty((rows, cols)), c.empty((cols,))
    c.relu_bias_backward(gd, zd, dx, db)
    ref_dx = O.relu_backward(g, z)
    got_dx = dx.numpy()
    assert_bits(got_dx, ref_dx, "dx")
    assert_sum(db.numpy(), ref_dx.astype(np.float64).sum(0), rows,
               ref32=seq_colsum32(ref_dx) if rows >= 1024 else None, what="db")
    # REFERENCE mode: the reference's full-sum-into-element-0 bias grad.
    dbr = c.empty((cols,))
    c.relu_bias_backward(gd, zd, None, dbr, mode=L.UNBROADCAST_REFERENCE)
    want = np.zeros(cols)
    want[0] = ref_dx.astype(np.float64).sum()
    got = dbr.numpy()
    assert_close(got[1:], want[1:], what="db ref rest")
    assert abs(got[0] - want[0]) <= 1e-5 + 1e-4 * np.abs(ref_dx).sum() ** 0.5 * 10, "db ref [0]"


def test_relu_bias_backward_accumulate_and_maskonly(hip_ctx, rng):
    rows, cols = 130, 300
    g, z = rand(rng, (rows, cols)), rand(rng, (rows, cols))
    g0x, g0b = rand(rng, (rows, cols)), rand(rng, cols)
    c = hip_ctx
    dx, db = c.to_device(g0x), c.to_device(g0b)
    c.relu_bias_backward(c.to_device(g), c.to_device(z), dx, db, accumulate=True)
    m = O.relu_backward(g, z)
    assert_bits(dx.numpy(), g0x + m, "dx acc")
    assert_close(db.numpy(), g0b.astype(np.float64) + m.astype(np.float64).sum(0), what="db acc")
    only = c.empty((rows, cols))
    c.relu_bias_backward(c.to_device(g), c.to_device(z), only, None)
    assert_bits(only.numpy(), m, "mask only")


SUM_CASES = [((4, 5), (5,)), ((4, 5), (1, 5)), ((4, 5), (4, 1)), ((3, 4, 5), (4, 1)),
             ((3, 4, 5), (3, 1, 5)), ((2, 3), (1,)), ((7,), (1,)), ((2, 3, 4), (2, 3, 4)),
             ((1000, 333), (333,)), ((17, 4096), (17, 1)), ((5, 1, 6), (1, 1, 6)),
             ((300000,), (1,))]


@pytest.mark.parametrize("gs,os_", SUM_CASES)
def test_sum_to_shape(hip_ctx, rng, gs, os_):
    say(f"sum_to_shape {gs}->{os_}")
    g = rand(rng, gs)
    c = hip_ctx
    out = c.empty(os_)
    c.sum_to_shape(c.to_device(g), out)
    assert_close(out.numpy(), O.sum_to_shape(g, os_), what=f"{gs}->{os_}")
    prev = rand(rng, os_)
    out2 = c.to_device(prev)
    c.sum_to_shape(c.to_device(g), out2, accumulate=True)
    assert_close(out2.numpy(), prev.astype(np.float64) + O.sum_to_shape(g, os_), what="acc")


def test_sum_to_shape_reference_mode(hip_ctx, rng):
    g = rand(rng, (64, 10))
    c = hip_ctx
    out = c.to_device(np.full(10, 3.0, np.float32))
    c.sum_to_shape(c.to_device(g), out, mode=L.UNBROADCAST_REFERENCE, accumulate=True)
    want = np.full(10, 3.0, np.float32)
    O.unbroadcast_reference_accumulate(g, want)
    assert_close(out.numpy(), want, what="reference acc")
    out = c.to_device(np.full(10, 3.0, np.float32))
    c.sum_to_shape(c.to_device(g), out, mode=L.UNBROADCAST_REFERENCE)
    want = np.zeros(10, np.float32)
    O.unbroadcast_reference_accumulate(g, want)
    assert_close(out.numpy(), want, what="reference fresh")


def test_sum_to_shape_rejects_bad_shape(hip_ctx):
    c = hip_ctx
    with pytest.raises(HipError) as e:
        c.sum_to_shape(c.zeros((4, 5)), c.zeros((3,)))
    assert e.value.code == L.E_SHAPE


# ---------------------------------------------------------------------------
# Elementwise backward
# ---------------------------------------------------------------------------

UNARY = [  # kind, oracle, input range, saved value from x, bit-exact?
    (L.RELU, O.relu_backward, (-2, 2), lambda x: x, True),
    (L.SIGMOID, O.sigmoid_backward, (-6, 6), lambda x: O.sigmoid(x), True),
    (L.TANH, O.tanh_backward, (-3, 3), lambda x: np.tanh(x).astype(np.float32), True),
    (L.EXP, O.exp_backward, (-3, 3), lambda x: np.exp(x).astype(np.float32), True),
    (L.LOG, O.log_backward, (0.1, 4), lambda x: x, True),
    (L.TAN, O.tan_backward, (-1.3, 1.3), lambda x: np.tan(x).astype(np.float32), True),
    (L.GELU, O.gelu_backward, (-5, 5), lambda x: x, False),
    (L.SQRT, O.sqrt_backward, (0.05, 9), lambda x: x, False),
    (L.SIN, O.sin_backward, (-6, 6), lambda x: x, False),
    (L.COS, O.cos_backward, (-6, 6), lambda x: x, False),
]


@pytest.mark.parametrize("n", [1, 5, 1000, 1 << 20])
@pytest.mark.parametrize("kind,orc,rng_,saved,exact", UNARY, ids=[str(u[0]) for u in UNARY])
def test_unary_backward(hip_ctx, rng, n, kind, orc, rng_, saved, exact):
    say(f"unary_backward kind={kind} n={n}")
    x = rng.uniform(*rng_, n).astype(np.float32)
    if kind == L.RELU:
        x[: min(3, n)] = 0.0
    v = saved(x)
    g = rand(rng, n)
    c = hip_ctx
    dx = c.empty(n)
    c.unary_backward(kind, c.to_device(g), c.to_device(v), dx)
    ref = orc(g, v)
    if exact:
        assert_bits(dx.numpy(), ref, f"kind {kind}")
    else:
        assert_close(dx.numpy(), ref, what=f"kind {kind}")


SPECIAL = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -1e-40, 1.0, -2.0, 3e38],
                   np.float32)


def _same_specials(got, want, what):
    """Same NaN positions, same infinities and zeros (with sign); finite values close."""
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn), f"{what}: NaN pattern"
    fin = np.isfinite(want) & (want != 0)
    assert np.array_equal(got[~gn & ~fin].view(np.uint32), want[~wn & ~fin].view(np.uint32)), \
        f"{what}: special values"
    assert np.allclose(got[fin], want[fin], rtol=1e-6, atol=0), f"{what}: finite values"


@pytest.mark.parametrize("expo", [2.5, 3.0, 2.0, 1.0, 0.0, 0.5, -1.5])
def test_pow_backward(hip_ctx, rng, expo):
    """Exponents whose power x^(n-1) takes a shortcut (n-1 = 2, 1, 0, -0.5) and two
    that use powf, against the oracle's glibc powf, special values included."""
    x = np.concatenate([rng.uniform(0.1, 3, 5000).astype(np.float32), SPECIAL])
    g = np.concatenate([rand(rng, 5000), np.ones(SPECIAL.size, np.float32)])
    c = hip_ctx
    dx = c.empty(x.size)
    c.unary_backward(L.POW, c.to_device(g), c.to_device(x), dx, param=expo)
    want = O.pow_backward(g, x, expo)
    got = dx.numpy()
    assert_close(got[:5000], want[:5000], what=f"pow {expo}")
    _same_specials(got[5000:], want[5000:], f"pow {expo} specials")


def test_sqrt_backward_specials(hip_ctx, rng):
    x = SPECIAL
    g = np.ones(x.size, np.float32)
    c = hip_ctx
    dx = c.empty(x.size)
    c.unary_backward(L.SQRT, c.to_device(g), c.to_device(x), dx)
    _same_specials(dx.numpy(), O.sqrt_backward(g, x), "sqrt specials")


def test_unary_accumulate_and_misaligned(hip_ctx, rng):
    n = 4099
    x, g, prev = rand(rng, n), rand(rng, n), rand(rng, n)
    c = hip_ctx
    xd, gd = c.to_device(x), c.to_device(g)
    base = c.to_device(np.concatenate([[0.0], prev]).astype(np.float32))
    dx = base.view(1, (n,))  # 4-byte offset: scalar path
    c.unary_backward(L.RELU, gd, xd, dx, accumulate=True)
    assert_bits(dx.numpy(), prev + O.relu_backward(g, x), "relu acc misaligned")


@pytest.mark.parametrize("kind", [L.ADD, L.SUB, L.MUL, L.DIV])
def test_binary_backward(hip_ctx, rng, kind):
    n = 100003
    g, x = rand(rng, n), rand(rng, n)
    y = rng.uniform(0.5, 2, n).astype(np.float32) * rng.choice([-1, 1], n).astype(np.float32)
    c = hip_ctx
    dx, dy = c.empty(n), c.empty(n)
    c.binary_backward(kind, c.to_device(g), c.to_device(x), c.to_device(y), dx, dy)
    if kind == L.ADD:
        rx, ry = g, g
    elif kind == L.SUB:
        rx, ry = O.sub_backward(g)
    elif kind == L.MUL:
        rx, ry = O.mul_backward(g, x, y)
    else:
        rx, ry = O.div_backward(g, x, y)
    assert_bits(dx.numpy(), rx, "dx")
    assert_bits(dy.numpy(), ry, "dy")


@pytest.mark.parametrize("kind", [L.ADD, L.SUB, L.MUL, L.DIV])
def test_binary_backward_accumulate_and_misaligned(hip_ctx, rng, kind):
    n = 4099
    g, x = rand(rng, n), rand(rng, n)
    y = rng.uniform(0.5, 2, n).astype(np.float32)
    px, py = rand(rng, n), rand(rng, n)
    rx, ry = {L.ADD: lambda: (g, g), L.SUB: lambda: O.sub_backward(g),
              L.MUL: lambda: O.mul_backward(g, x, y), L.DIV: lambda: O.div_backward(g, x, y)}[kind]()
    c = hip_ctx
    for off in (0, 1):  # 0: float4 path; 1: 4-byte offset views, scalar path
        bx = c.to_device(np.concatenate([np.zeros(off), px]).astype(np.float32))
        by = c.to_device(np.concatenate([np.zeros(off), py]).astype(np.float32))
        dx, dy = bx.view(off, (n,)), by.view(off, (n,))
        c.binary_backward(kind, c.to_device(g), c.to_device(x), c.to_device(y), dx, dy,
                          accumulate=True)
        assert_bits(dx.numpy(), px + rx, f"dx acc off={off}")
        assert_bits(dy.numpy(), py + ry, f"dy acc off={off}")


def test_fill_and_mse_accumulate_and_misaligned(hip_ctx, rng):
    c = hip_ctx
    g0 = c.to_device(np.array([0.7], np.float32))
    n = 4099
    prev, p, t = rand(rng, n), rand(rng, n), rand(rng, n)
    rp, rt = O.mse_backward(np.float32(0.7), p, t)
    for off in (0, 1):
        base = c.to_device(np.concatenate([np.zeros(off), prev]).astype(np.float32))
        dx = base.view(off, (n,))
        c.fill_grad(g0, dx, divide_by_n=True, accumulate=True)
        assert_bits(dx.numpy(), prev + O.mean_backward(np.float32(0.7), (n,)), f"fill off={off}")
        bp = c.to_device(np.concatenate([np.zeros(off), prev]).astype(np.float32))
        bt = c.to_device(np.concatenate([np.zeros(off), prev]).astype(np.float32))
        dp, dt = bp.view(off, (n,)), bt.view(off, (n,))
        c.mse_backward(g0, c.to_device(p), c.to_device(t), dp, dt, accumulate=True)
        assert_bits(dp.numpy(), prev + rp, f"mse dp acc off={off}")
        assert_bits(dt.numpy(), prev + rt, f"mse dt acc off={off}")


def test_fill_grad_and_mse(hip_ctx, rng):
    c = hip_ctx
    g0 = c.to_device(np.array([0.7], np.float32))
    n = 12345
    dx = c.empty(n)
    c.fill_grad(g0, dx)
    assert_bits(dx.numpy(), O.sum_backward(np.float32(0.7), (n,)), "sum bwd")
    c.fill_grad(g0, dx, divide_by_n=True)
    assert_bits(dx.numpy(), O.mean_backward(np.float32(0.7), (n,)), "mean bwd")
    p, t = rand(rng, n), rand(rng, n)
    dp, dt = c.empty(n), c.empty(n)
    c.mse_backward(g0, c.to_device(p), c.to_device(t), dp, dt)
    rp, rt = O.mse_backward(np.float32(0.7), p, t)
    assert_bits(dp.numpy(), rp, "mse dp")
    assert_bits(dt.numpy(), rt, "mse dt")
    # reference KAT tests/autograd_loss.rs:5-37
    one = c.to_device(np.array([1.0], np.float32))
    dp3 = c.empty(3)
    c.mse_backward(one, c.to_device(np.array([1, 2, 3.0])), c.to_device(np.array([1, 2, 5.0])), dp3)
    got = dp3.numpy()
    assert got[0] == 0.0 and abs(got[2] + 1.333333) < 1e-5


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 5), (64, 64), (68, 132), (4, 4096),
                                       (4096, 2048), (130, 4), (33, 31), (64, 256),
                                       (68, 260), (196, 1020), (2052, 4)])
def test_transpose(hip_ctx, rng, rows, cols):
    """numrs_hip_transpose (ops/shape/transpose.rs:9-88): the register form (64x256
    workgroups of 4x4 lane blocks, ragged at both edges in 68x260 and 196x1020) from
    64x256 up, 128x128 or 64x64 float4 LDS tiles below it when both dimensions are
    multiples of 4, 32x32 tiles otherwise; a copy, so bit-exact."""
    x = rand(rng, (rows, cols))
    c = hip_ctx
    y, xd = c.empty((cols, rows)), c.to_device(x)  # held for the call: a temporary is freed at once
    c._check(L.load().numrs_hip_transpose(c.handle, xd.ptr, y.ptr, rows, cols))
    assert_bits(y.numpy(), np.ascontiguousarray(x.T), f"transpose {rows}x{cols}")


@pytest.mark.parametrize("n", [1, 3, 4, 5, 1023, 4096, 100003, 1 << 22])
def test_full_sum_mean_mse(hip_ctx, rng, n):
    """numrs_hip_sum / mean / mse_loss (ops.rs:214-278) over aligned and offset inputs."""
    c = hip_ctx
    x, t = rand(rng, n), rand(rng, n)
    out = c.empty((1,))
    fn = L.load()
    tol = 1e-6 * np.sqrt(n) + 1e-6
    for off in (0, 1):
        xb = c.to_device(np.concatenate([np.zeros(off), x]).astype(np.float32))
        tb = c.to_device(np.concatenate([np.zeros(off), t]).astype(np.float32))
        xd, td = xb.view(off, (n,)), tb.view(off, (n,))
        c._check(fn.numrs_hip_sum(c.handle, xd.ptr, n, 0, out.ptr))
        assert abs(out.numpy()[0] - x.astype(np.float64).sum()) <= tol * 4, (n, off, "sum")
        c._check(fn.numrs_hip_sum(c.handle, xd.ptr, n, 1, out.ptr))
        assert abs(out.numpy()[0] - x.astype(np.float64).mean()) <= tol * 4 / n + 1e-7, (n, off)
        c._check(fn.numrs_hip_mse_loss(c.handle, xd.ptr, td.ptr, n, out.ptr))
        want = ((x.astype(np.float64) - t) ** 2).mean()
        assert abs(out.numpy()[0] - want) <= 1e-5 * want + 1e-7, (n, off, "mse")


@pytest.mark.parametrize("n,off", [(1 << 20, 0), (12345, 0), (4099, 1), (3, 0)])
def test_copy(hip_ctx, rng, n, off):
    """numrs_hip_copy: the float4 kernel (aligned) and the fallback (offset views)."""
    c = hip_ctx
    x = rand(rng, n + off)
    src, dst = c.to_device(x), c.zeros(n + off)
    c.copy(dst.view(off, (n,)), src.view(off, (n,)))
    got = dst.numpy()
    assert_bits(got[off:], x[off:], "copy")
    assert np.all(got[:off] == 0)

# ---------------------------------------------------------------------------
# Row-wise: softmax-CE, softmax backward, argmax
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("B,C", [(1, 2), (64, 10), (7, 1000), (256, 129), (33, 4), (300, 2048),
                                 (5, 2052), (4096, 1024)])
def test_softmax_ce_backward(hip_ctx, rng, B, C):
    say(f"softmax_ce_backward {B}x{C}")
    x = rand(rng, (B, C), 3.0)
    labels = rng.integers(0, C, B).astype(np.int32)
    onehot = np.eye(C, dtype=np.float32)[labels]
    c = hip_ctx
    g0 = c.to_device(np.array([1.0], np.float32))
    xd = c.to_device(x)
    d1, d2 = c.empty((B, C)), c.empty((B, C))
    c.softmax_ce_backward(g0, xd, d1, onehot=c.to_device(onehot))
    c.softmax_ce_backward(g0, xd, d2, labels=c.to_device(labels))
    ref = O.cross_entropy_backward(1.0, x, onehot)
    assert_close(d1.numpy(), ref, what="onehot")
    assert_bits(d2.numpy(), d1.numpy(), "labels == onehot")


UNARY_FWD_KINDS = [L.RELU, L.SIGMOID, L.TANH, L.EXP, L.LOG, L.GELU, L.SQRT, L.SIN, L.COS, L.TAN,
                   L.POW]


@pytest.mark.parametrize("kind", UNARY_FWD_KINDS)
@pytest.mark.parametrize("n", [4099, 100003, (1 << 23) + 5])
def test_unary_forward_vector_equals_scalar(hip_ctx, rng, kind, n):
    """numrs_hip_unary_forward on 16-byte aligned buffers (float4 groups, the
    streaming access mode from 2^23 elements, an element-wise tail) gives the
    same bits as on misaligned ones (the element-per-thread kernel), and both
    match numpy's float64 value to float32 rounding."""
    say(f"unary_forward kind {kind} n={n}")
    x = rng.uniform(-3, 3, n).astype(np.float32)
    if kind in (L.LOG, L.SQRT, L.POW):
        x = np.abs(x) + np.float32(0.01)
    x[:4] = [0.0, -0.0, 1.0, -1.0] if kind not in (L.LOG, L.SQRT, L.POW) else [0.5, 1.0, 2.0, 3.0]
    c = hip_ctx
    lib = L.load()
    xa, ya = c.to_device(x), c.empty((n,))
    xm_base = c.to_device(np.concatenate([np.zeros(1, np.float32), x]))
    ym_base = c.empty((n + 1,))
    xm, ym = xm_base.view(1, (n,)), ym_base.view(1, (n,))
    p = 1.7
    assert lib.numrs_hip_unary_forward(c.handle, kind, xa.ptr, ya.ptr, n, p) == 0
    assert lib.numrs_hip_unary_forward(c.handle, kind, xm.ptr, ym.ptr, n, p) == 0
    got = ya.numpy()
    assert_bits(got, ym.numpy(), f"kind {kind}: float4 path vs element path")
    x64 = x.astype(np.float64)
    ref = {L.RELU: lambda: np.maximum(x64, 0), L.SIGMOID: lambda: 1 / (1 + np.exp(-x64)),
           L.TANH: lambda: np.tanh(x64), L.EXP: lambda: np.exp(x64), L.LOG: lambda: np.log(x64),
           L.GELU: lambda: (0.5 * x64 * (1 + np.vectorize(math.erf)(x64 / math.sqrt(2)))
                            if n < 200000 else None),
           L.SQRT: lambda: np.sqrt(x64), L.SIN: lambda: np.sin(x64), L.COS: lambda: np.cos(x64),
           L.TAN: lambda: np.tan(x64), L.POW: lambda: x64 ** np.float64(np.float32(p))}[kind]()
    if ref is not None:
        assert_close(got, ref, abs_tol=2e-6, rel_tol=4e-6, what=f"kind {kind} vs float64")


@pytest.mark.parametrize("kind", [L.ADD, L.SUB, L.MUL, L.DIV])
@pytest.mark.parametrize("n", [4099, 100003, (1 << 23) + 7])
@pytest.mark.parametrize("form", ["same", "b_scalar", "a_scalar"])
def test_binary_forward_vector_equals_scalar(hip_ctx, rng, kind, n, form):
    """numrs_hip_binary_forward over equal shapes or a one-element operand:
    16-byte aligned buffers (float4 groups) give the same bits as misaligned
    views (one element per thread), and both equal numpy's float32 result."""
    say(f"binary_forward kind {kind} n={n} {form}")
    a = rng.uniform(-3, 3, n).astype(np.float32)
    b = (rng.uniform(0.5, 2.0, n) * rng.choice([-1.0, 1.0], n)).astype(np.float32)
    if form == "b_scalar":
        b = b[:1].copy()
    if form == "a_scalar":
        a = a[:1].copy()
    c = hip_ctx
    lib = L.load()

    def run(aligned):
        def dev(v):
            if aligned:
                return c.to_device(v), None
            base = c.to_device(np.concatenate([np.zeros(1, np.float32), v]))
            return base.view(1, v.shape), base
        (ad, _ka), (bd, _kb) = dev(a), dev(b)
        out_base = c.empty((n + 1,))
        out = out_base if aligned else out_base.view(1, (n,))
        ash, bsh = (ctypes.c_int64 * 1)(a.size), (ctypes.c_int64 * 1)(b.size)
        assert lib.numrs_hip_binary_forward(c.handle, kind, ad.ptr, ash, 1, bd.ptr, bsh, 1,
                                            out.ptr) == 0
        return out.numpy()[:n]

    got, ref_scalar = run(True), run(False)
    assert_bits(got, ref_scalar, f"kind {kind} {form}: float4 path vs element path")
    want = {L.ADD: np.add, L.SUB: np.subtract, L.MUL: np.multiply, L.DIV: np.divide}[kind](a, b)
    assert_bits(got, np.broadcast_to(want, (n,)), f"kind {kind} {form}: vs numpy float32")


LN_CASES = [(1, 1), (7, 5), (33, 64), (130, 1000), (9, 2048), (5, 2047), (1030, 300),
            (4096, 512)]


@pytest.mark.parametrize("rows,cols", LN_CASES + [(3, 2056), (2, 4096), (64, 256), (8, 1024)])
def test_layernorm_forward(hip_ctx, rng, rows, cols):
    """Register-resident rows (cols % 4 == 0, up to 2048) and the looped
    kernel (other widths) against the float64 statistics."""
    say(f"layernorm_forward {rows}x{cols}")
    x = rand(rng, (rows, cols)) + 3.0  # an offset the mean must remove
    gamma = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    beta = rand(rng, cols)
    x64 = x.astype(np.float64)
    mu = x64.mean(1, keepdims=True)
    rs = 1.0 / np.sqrt(((x64 - mu) ** 2).mean(1, keepdims=True) + 1e-5)
    want = (x64 - mu) * rs * gamma + beta
    c = hip_ctx
    xd, gd, bd = c.to_device(x), c.to_device(gamma), c.to_device(beta)
    y, m, r = c.empty((rows, cols)), c.empty((rows,)), c.empty((rows,))
    c._check(L.load().numrs_hip_layernorm_forward(c.handle, xd.ptr, gd.ptr, bd.ptr, y.ptr, m.ptr,
                                                  r.ptr, rows, cols, 1e-5))
    assert_close(y.numpy(), want, what="y")
    assert_close(m.numpy(), mu[:, 0], what="mean")
    assert_close(r.numpy(), rs[:, 0], what="rstd")
    # the oracle's LayerNorm (float64 inside, rounded to fp32 on output)
    want_o, _, _ = O.layernorm_fwd(x, gamma, beta)
    assert_close(y.numpy(), want_o, what="y vs oracle")


@pytest.mark.parametrize("rows,cols", LN_CASES)
def test_layernorm_backward(hip_ctx, rng, rows, cols):
    say(f"layernorm_backward {rows}x{cols}")
    x, g = rand(rng, (rows, cols)), rand(rng, (rows, cols))
    gamma = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    _, mean, rstd = O.layernorm_fwd(x, gamma, np.zeros(cols, np.float32))
    want_dx, want_dg, want_db = O.layernorm_backward(g, x, gamma)
    c = hip_ctx
    xd, gd, gmd = c.to_device(x), c.to_device(g), c.to_device(gamma)
    md, rd = c.to_device(mean), c.to_device(rstd)
    fn = L.load().numrs_hip_layernorm_backward

    def run(dx, dg, db, acc=(0, 0, 0)):
        c._check(fn(c.handle, gd.ptr, xd.ptr, gmd.ptr, md.ptr, rd.ptr,
                    dx.ptr if dx is not None else None, dg.ptr if dg is not None else None,
                    db.ptr if db is not None else None, rows, cols, *acc))

    dx, dg, db = c.empty((rows, cols)), c.empty((cols,)), c.empty((cols,))
    run(dx, dg, db)
    assert_close(dx.numpy(), want_dx, abs_tol=2e-5, rel_tol=1e-3, what="dx")
    assert_close(dg.numpy(), want_dg, abs_tol=2e-5, rel_tol=1e-3, what="dgamma")
    assert_close(db.numpy(), want_db, abs_tol=2e-5, rel_tol=1e-3, what="dbeta")
    # accumulate into existing grads; dbeta alone; dgamma alone
    base_dx, base_dg = rand(rng, (rows, cols)), rand(rng, cols)
    dx2, dg2 = c.to_device(base_dx), c.to_device(base_dg)
    run(dx2, dg2, None, acc=(1, 1, 0))
    assert_close(dx2.numpy(), base_dx.astype(np.float64) + want_dx, abs_tol=2e-5, rel_tol=1e-3,
                 what="dx acc")
    assert_close(dg2.numpy(), base_dg.astype(np.float64) + want_dg, abs_tol=2e-5, rel_tol=1e-3,
                 what="dgamma acc")
    db3 = c.empty((cols,))
    run(None, None, db3)
    assert_close(db3.numpy(), want_db, abs_tol=2e-5, rel_tol=1e-3, what="dbeta only")


@pytest.mark.parametrize("rows,cols", [(1, 1), (5, 7), (2048, 256), (3, 5000), (17, 1000),
                                       (9, 2048), (6, 12)])
def test_softmax_backward(hip_ctx, rng, rows, cols):
    y = O.softmax_rows(rand(rng, (rows, cols), 2.0))
    g = rand(rng, (rows, cols))
    c = hip_ctx
    dx = c.empty((rows, cols))
    c.softmax_backward(c.to_device(y), c.to_device(g), dx)
    want = O.softmax_backward(y, g, f64=True)
    assert_close(dx.numpy(), want)
    # in place (g and dx the same buffer), accumulate into it
    gd = c.to_device(g)
    c.softmax_backward(c.to_device(y), gd, gd, accumulate=True)
    assert_close(gd.numpy(), g.astype(np.float64) + want, what="in place acc")


def test_argmax_rows(hip_ctx, rng):
    say("argmax")
    c = hip_ctx
    cases = [rand(rng, (64, 10)), rand(rng, (5, 1000)),
             np.array([[1, 3, 2, 3, 1], [3, 1, 4, 1, 5], [-5, -2, -3, -4, -2]], np.float32),
             np.array([[np.nan, 1, 2], [1, np.nan, 0], [0, 2, np.nan], [0.0, -0.0, 0.0],
                       [2, 2, 2], [np.nan, np.nan, np.nan]], np.float32),
             rng.integers(0, 3, (300, 130)).astype(np.float32),
             # register-resident path (cols % 4 == 0): ties, NaNs, +-0
             rng.integers(0, 3, (300, 128)).astype(np.float32),
             np.array([[np.nan, 1, 2, 2, 0, 1, 2, 1], [1, 2, np.nan, 2, 0, 2, 1, 0],
                       [0, 2, 1, 2, 1, 2, 1, np.nan], [0.0, -0.0, 0.0, -0.0, 0, 0, -0.0, 0],
                       [3, 3, 3, 3, 3, 3, 3, 3], [np.nan] * 8], np.float32),
             rand(rng, (33, 2048)), rng.integers(0, 2, (7, 1000)).astype(np.float32)]
    # Wide register-resident rows (four and eight float4 groups per lane) with
    # ties spread over every lane and NaNs in some rows: the wave's combine of
    # (value, index) pairs across lanes decides these.
    for w in (1024, 2048):
        t = rng.integers(0, 4, (96, w)).astype(np.float32)
        t[rng.random(t.shape) < 0.002] = np.nan
        cases.append(t)
    for x in cases:
        for tie_last in (False, True):
            idx = c.empty((x.shape[0],), np.int32)
            c.argmax_rows(c.to_device(x), idx, tie_last=tie_last)
            assert idx.numpy().tolist() == O.argmax_rows(x, tie_last).tolist(), (x, tie_last)


# ---------------------------------------------------------------------------
# Optimizers
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("mu,wd", [(0.0, 0.0), (0.9, 0.0), (0.0, 0.1), (0.9, 1e-4)])
def test_sgd_step(hip_ctx, rng, mu, wd):
    n = 101770  # the C1 MLP parameter count
    p, g = rand(rng, n), rand(rng, n)
    v = np.zeros(n, np.float32)
    c = hip_ctx
    pd, gd, vd = c.to_device(p), c.to_device(g), c.to_device(v)
    for _ in range(3):
        c.sgd_step(pd, gd, vd if mu else None, lr=0.01, mu=mu, wd=wd)
        O.sgd_step(p, g, v if mu else None, 0.01, mu, wd)
    assert_bits(pd.numpy(), p, "p")
    if mu:
        assert_bits(vd.numpy(), v, "v")


@pytest.mark.parametrize("n,wd", [(1, 0.0), (1003, 0.0), (1 << 24, 0.0), (4097, 0.01)])
def test_adam_step(hip_ctx, rng, n, wd):
    say(f"adam n={n} wd={wd}")
    p, g = rand(rng, n), rand(rng, n)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    c = hip_ctx
    pd, gd, md, vd = c.to_device(p), c.to_device(g), c.to_device(m), c.to_device(v)
    steps = 2 if n > 100000 else 11
    for t in range(1, steps + 1):
        c.adam_step(pd, gd, md, vd, t, lr=1e-3, wd=wd)
        O.adam_step(p, g, m, v, t, lr=1e-3, wd=wd)
    assert_bits(pd.numpy(), p, "p")
    assert_bits(md.numpy(), m, "m")
    assert_bits(vd.numpy(), v, "v")


def test_adam_kat(hip_ctx):
    # tests/autograd/optim/adam.rs:8-62
    c = hip_ctx
    p, g = c.to_device(np.array([1.0], np.float32)), c.to_device(np.array([1.0], np.float32))
    m, v = c.zeros(1), c.zeros(1)
    c.adam_step(p, g, m, v, 1, lr=0.1)
    assert abs(p.numpy()[0] - 0.9) < 1e-5
    c.adam_step(p, g, m, v, 2, lr=0.1)
    assert abs(p.numpy()[0] - 0.8) < 1e-4


def test_error_paths(hip_ctx):
    c = hip_ctx
    x = c.zeros(4)
    with pytest.raises(HipError) as e:
        c.unary_backward(99, x, x, x)
    assert e.value.code == L.E_INVALID
    with pytest.raises(HipError):
        c.adam_step(x, x, x, x, 0)
    with pytest.raises(HipError):
        c.softmax_ce_backward(x.view(0, (1,)), x.view(0, (2, 2)), x.view(0, (2, 2)))


@pytest.mark.parametrize("M,K,N", [(4096, 512, 512), (4096, 256, 384), (8192, 128, 64),
                                   (3000, 130, 70), (1024, 1024, 1024), (2048, 1024, 512)])
@pytest.mark.parametrize("acc", [False, True])
def test_matmul_backward_split_k(hip_ctx, rng, M, K, N, acc):
    # Weight-gradient shapes: dB = A^T dC has few output tiles and a long
    # reduction over M, so it runs split-K (deterministic partials + reduce).
    say(f"split-k matmul_backward M={M} K={K} N={N} acc={acc}")
    A, B, dC = rand(rng, (M, K)), rand(rng, (K, N)), rand(rng, (M, N))
    ga, gb = rand(rng, (M, K)), rand(rng, (K, N))
    c = hip_ctx
    dA = c.to_device(ga) if acc else c.empty((M, K))
    dB = c.to_device(gb) if acc else c.empty((K, N))
    c.matmul_backward(c.to_device(dC), c.to_device(A), c.to_device(B), dA, dB, accumulate=acc)
    _, rb = O.matmul_backward(dC, A, B, need_a=False, f64=True)
    _, rb32 = O.matmul_backward(dC, A, B, need_a=False)
    base_b = gb.astype(np.float64) if acc else 0.0
    assert_contraction(dB.numpy(), base_b + rb, M, ref32=None if acc else rb32, what="dB")
    ra, _ = O.matmul_backward(dC, A, B, need_b=False, f64=True, rows_a=(0, 64))
    base_a = ga[:64].astype(np.float64) if acc else 0.0
    assert_contraction(dA.numpy()[:64], base_a + ra[:64], N, what="dA rows")
    # determinism: the same call again gives identical bits
    dA2 = c.to_device(ga) if acc else c.empty((M, K))
    dB2 = c.to_device(gb) if acc else c.empty((K, N))
    c.matmul_backward(c.to_device(dC), c.to_device(A), c.to_device(B), dA2, dB2, accumulate=acc)
    assert_bits(dB2.numpy(), dB.numpy(), "split-k determinism")
    assert_bits(dA2.numpy(), dA.numpy(), "split-k determinism (dA)")
    # dB alone: its own split plan (the pair's plan balances both products,
    # so the rounding may differ from the pair's dB), same tolerance.
    dB3 = c.to_device(gb) if acc else c.empty((K, N))
    c.matmul_backward(c.to_device(dC), c.to_device(A), c.to_device(B), None, dB3, accumulate=acc)
    assert_contraction(dB3.numpy(), base_b + rb, M, ref32=None if acc else rb32, what="dB alone")


def test_matmul_forward_split_k_long_reduction(hip_ctx, rng):
    A, B = rand(rng, (64, 8192)), rand(rng, (8192, 64))
    c = hip_ctx
    C = c.empty((64, 64))
    c.matmul(c.to_device(A), c.to_device(B), C)
    assert_contraction(C.numpy(), A.astype(np.float64) @ B.astype(np.float64), 8192)


# (4096, 512, 2048), (4096, 2048, 512), (4096, 512, 512) and (4096, 512, 1536)
# (the packed q/k/v projection) are the C4 block's Linear shapes: the streamed
# 256 x 128 path with split-K ranges planned per product (dx and dW in one
# grid, each reduced in split order).  The bias gradient (CORRECT mode) is
# formed by the split-reduce launch for float4 columns and up to 8192 rows:
# (8192, 64, 100) ends on a partial 16-column group; (9000, 32, 64) and
# (130, 96, 18) take the two-pass column reduce.
@pytest.mark.parametrize("T,fin,fout", [(64, 784, 128), (64, 128, 10), (4096, 512, 2048),
                                        (4096, 2048, 512), (4096, 512, 512), (4096, 512, 1536),
                                        (8192, 64, 100), (9000, 32, 64), (130, 96, 18),
                                        (33, 17, 5)])
def test_linear_forward_backward(hip_ctx, rng, T, fin, fout):
    # Linear::forward (nn.rs:217-235) and the grads its Transpose/MatMul/Add
    # nodes produce (backward.rs:43-54, 113-149, 305-312).
    say(f"linear T={T} in={fin} out={fout}")
    x, W, b, g = rand(rng, (T, fin)), rand(rng, (fout, fin)), rand(rng, fout), rand(rng, (T, fout))
    c = hip_ctx
    xd, Wd, bd, gd = (c.to_device(a) for a in (x, W, b, g))
    y = c.empty((T, fout))
    rc = L.load().numrs_hip_linear_forward(c.handle, xd.ptr, Wd.ptr, bd.ptr, y.ptr, T, fin, fout)
    assert rc == 0
    ref_y = O.matmul_f64(x, O.transpose(W)).astype(np.float64) + b
    assert_contraction(y.numpy(), ref_y, fin, what="y")
    prev = {k: rand(rng, s) for k, s in (("dx", (T, fin)), ("dW", (fout, fin)), ("db", fout))}
    for acc in ((0, 0, 0), (1, 0, 1), (0, 1, 0)):
        dx, dW, db = (c.to_device(prev[k]) for k in ("dx", "dW", "db"))
        rc = L.load().numrs_hip_linear_backward(c.handle, gd.ptr, xd.ptr, Wd.ptr, dx.ptr, dW.ptr,
                                                db.ptr, T, fin, fout, *acc, L.UNBROADCAST_CORRECT)
        assert rc == 0
        rdx, rdwt = O.matmul_backward(g, x, O.transpose(W), f64=True)
        base = [prev[k].astype(np.float64) if a else 0.0 for k, a in zip(("dx", "dW", "db"), acc)]
        assert_contraction(dx.numpy(), base[0] + rdx, fout, what=f"dx {acc}")
        assert_contraction(dW.numpy(), base[1] + O.transpose(rdwt), T, what=f"dW {acc}")
        assert_sum(db.numpy(), base[2] + g.astype(np.float64).sum(0), T,
                   ref32=(base[2] + seq_colsum32(g)) if T >= 1024 else None, what=f"db {acc}")
    # REFERENCE-mode bias gradient: full sum into db[0]
    db = c.to_device(prev["db"])
    rc = L.load().numrs_hip_linear_backward(c.handle, gd.ptr, xd.ptr, Wd.ptr, None, None, db.ptr,
                                            T, fin, fout, 0, 0, 0, L.UNBROADCAST_REFERENCE)
    assert rc == 0
    want = np.zeros(fout, np.float32)
    O.unbroadcast_reference_accumulate(g, want)
    got = db.numpy()
    assert np.all(got[1:] == 0) and np.all(want[1:] == 0), "db reference: only element 0 is set"
    # db[0] is a length-T*fout fp32 sum: numrs's own 8-lane fp32 result carries a
    # rounding error of the same order as the difference to ours, so both are
    # compared with the float64 sum, and ours must be at least as close.
    exact = g.astype(np.float64).sum()
    e_gpu, e_ref = abs(float(got[0]) - exact), abs(float(want[0]) - exact)
    assert e_gpu <= max(e_ref, 1e-4 + 1e-6 * abs(exact)), (
        f"db reference: |gpu - exact| {e_gpu:.3e} vs numrs fp32 sum {e_ref:.3e}")


# Linear followed by ReLU as one op.  (64, 784, 128), (64, 128, 10), (130,
# 96, 18) and (33, 17, 5) take the tiny kernel (ReLU in the forward epilogue,
# the backward mask applied as g is loaded, dx/dW/db in one launch);
# (4096, 512, 512) the Linear path with the ReLU and the mask as passes of
# their own.  Each result must equal the two-op composition bit for bit.
@pytest.mark.parametrize("T,fin,fout", [(64, 784, 128), (64, 128, 10), (130, 96, 18),
                                        (33, 17, 5), (4096, 512, 512)])
def test_linear_relu_forward_backward(hip_ctx, rng, T, fin, fout):
    say(f"linear+relu T={T} in={fin} out={fout}")
    lib = L.load()
    x, W, b, g = rand(rng, (T, fin)), rand(rng, (fout, fin)), rand(rng, fout), rand(rng, (T, fout))
    c = hip_ctx
    xd, Wd, bd, gd = (c.to_device(a) for a in (x, W, b, g))
    y, y2 = c.empty((T, fout)), c.empty((T, fout))
    assert lib.numrs_hip_linear_relu_forward(c.handle, xd.ptr, Wd.ptr, bd.ptr, y.ptr, T, fin,
                                             fout) == 0
    assert lib.numrs_hip_linear_forward(c.handle, xd.ptr, Wd.ptr, bd.ptr, y2.ptr, T, fin, fout) == 0
    assert lib.numrs_hip_unary_forward(c.handle, L.RELU, y2.ptr, y2.ptr, T * fout, 0.0) == 0
    yv = y.numpy()
    assert np.array_equal(yv, y2.numpy()), "fused forward != linear + relu"
    ref_y = O.matmul_f64(x, O.transpose(W)).astype(np.float64) + b
    assert_contraction(yv, np.maximum(ref_y, 0.0), fin, what="y")
    assert (yv >= 0).all()
    # the mask is the GPU's own y > 0, so sign flips at |pre| ~ rounding do not matter
    gm = np.where(yv > 0, g, 0.0).astype(np.float32)
    gmd = c.to_device(gm)
    prev = {k: rand(rng, s) for k, s in (("dx", (T, fin)), ("dW", (fout, fin)), ("db", fout))}
    for acc in ((0, 0, 0), (1, 0, 1), (0, 1, 0)):
        dx, dW, db = (c.to_device(prev[k]) for k in ("dx", "dW", "db"))
        assert lib.numrs_hip_linear_relu_backward(c.handle, gd.ptr, y.ptr, xd.ptr, Wd.ptr, dx.ptr,
                                                  dW.ptr, db.ptr, T, fin, fout, *acc,
                                                  L.UNBROADCAST_CORRECT) == 0
        dx2, dW2, db2 = (c.to_device(prev[k]) for k in ("dx", "dW", "db"))
        assert lib.numrs_hip_linear_backward(c.handle, gmd.ptr, xd.ptr, Wd.ptr, dx2.ptr, dW2.ptr,
                                             db2.ptr, T, fin, fout, *acc,
                                             L.UNBROADCAST_CORRECT) == 0
        for name, a, b2 in (("dx", dx, dx2), ("dW", dW, dW2), ("db", db, db2)):
            assert np.array_equal(a.numpy(), b2.numpy()), f"{name} {acc}: fused != composition"
        rdx, rdwt = O.matmul_backward(gm, x, O.transpose(W), f64=True)
        base = [prev[k].astype(np.float64) if a else 0.0 for k, a in zip(("dx", "dW", "db"), acc)]
        assert_contraction(dx.numpy(), base[0] + rdx, fout, what=f"dx {acc}")
        assert_contraction(dW.numpy(), base[1] + O.transpose(rdwt), T, what=f"dW {acc}")
        assert_sum(db.numpy(), base[2] + gm.astype(np.float64).sum(0), T, what=f"db {acc}")
    # only some of the gradients, and the REFERENCE-mode bias (full sum in db[0])
    dW = c.to_device(prev["dW"])
    assert lib.numrs_hip_linear_relu_backward(c.handle, gd.ptr, y.ptr, xd.ptr, Wd.ptr, None,
                                              dW.ptr, None, T, fin, fout, 0, 0, 0,
                                              L.UNBROADCAST_CORRECT) == 0
    rdx, rdwt = O.matmul_backward(gm, x, O.transpose(W), f64=True)
    assert_contraction(dW.numpy(), O.transpose(rdwt), T, what="dW alone")
    db, db2 = c.to_device(prev["db"]), c.to_device(prev["db"])
    assert lib.numrs_hip_linear_relu_backward(c.handle, gd.ptr, y.ptr, xd.ptr, Wd.ptr, None, None,
                                              db.ptr, T, fin, fout, 0, 0, 0,
                                              L.UNBROADCAST_REFERENCE) == 0
    assert lib.numrs_hip_relu_bias_backward(c.handle, gd.ptr, y.ptr, None, db2.ptr, T, fout,
                                            L.UNBROADCAST_REFERENCE, 0) == 0
    assert np.array_equal(db.numpy(), db2.numpy()), "db reference mode"
    assert np.all(db.numpy()[1:] == 0)


# y = res + (x W^T + b) with the residual in the epilogue of each GEMM path:
# tiny (64, 784, 128) and (130, 96, 18), streamed (4096, 512, 512), streamed
# with split-K (4096, 2048, 512: the epilogue runs in the split reduction),
# the wide 128 x 192 tile (4096, 512, 1536), the 128 x 128 path (1000, 300,
# 136).  Bit for bit the Linear forward followed by an add; also with res
# aliasing y.
@pytest.mark.parametrize("T,fin,fout", [(64, 784, 128), (130, 96, 18), (4096, 512, 512),
                                        (4096, 2048, 512), (4096, 512, 1536), (1000, 300, 136)])
def test_linear_residual_forward(hip_ctx, rng, T, fin, fout):
    say(f"linear+residual T={T} in={fin} out={fout}")
    lib = L.load()
    x, W, b, r = rand(rng, (T, fin)), rand(rng, (fout, fin)), rand(rng, fout), rand(rng, (T, fout))
    c = hip_ctx
    xd, Wd, bd, rd = (c.to_device(a) for a in (x, W, b, r))
    y, f = c.empty((T, fout)), c.empty((T, fout))
    assert lib.numrs_hip_linear_residual_forward(c.handle, xd.ptr, Wd.ptr, bd.ptr, rd.ptr, y.ptr,
                                                 T, fin, fout) == 0
    assert lib.numrs_hip_linear_forward(c.handle, xd.ptr, Wd.ptr, bd.ptr, f.ptr, T, fin, fout) == 0
    want = r + f.numpy()  # fp32 add, as the add kernel rounds it
    assert np.array_equal(y.numpy(), want), "fused residual != linear + add"
    ref = O.matmul_f64(x, O.transpose(W)).astype(np.float64) + b + r
    assert_contraction(y.numpy(), ref, fin, what="y")
    # in place: res is y
    assert lib.numrs_hip_linear_residual_forward(c.handle, xd.ptr, Wd.ptr, bd.ptr, rd.ptr, rd.ptr,
                                                 T, fin, fout) == 0
    assert np.array_equal(rd.numpy(), want), "residual aliasing y"


# Linear followed by GELU as one op, the pre-activation stored by the
# epilogue: tiny (64, 784, 128) and (33, 17, 5), streamed (4096, 512, 2048:
# the C4 FFN's first projection), streamed with split-K (4096, 2048, 512),
# the wide 128 x 192 tile (4096, 512, 1536), the 128 x 128 path (1000, 300,
# 136).  Bit for bit the two-op composition.
@pytest.mark.parametrize("T,fin,fout", [(64, 784, 128), (33, 17, 5), (4096, 512, 2048),
                                        (4096, 2048, 512), (4096, 512, 1536), (1000, 300, 136)])
def test_linear_gelu_forward_backward(hip_ctx, rng, T, fin, fout):
    say(f"linear+gelu T={T} in={fin} out={fout}")
    lib = L.load()
    x, W, b, g = rand(rng, (T, fin)), rand(rng, (fout, fin)), rand(rng, fout), rand(rng, (T, fout))
    c = hip_ctx
    xd, Wd, bd, gd = (c.to_device(a) for a in (x, W, b, g))
    y, pre, y2, pre2 = (c.empty((T, fout)) for _ in range(4))
    assert lib.numrs_hip_linear_gelu_forward(c.handle, xd.ptr, Wd.ptr, bd.ptr, y.ptr, pre.ptr, T,
                                             fin, fout) == 0
    assert lib.numrs_hip_linear_forward(c.handle, xd.ptr, Wd.ptr, bd.ptr, pre2.ptr, T, fin,
                                        fout) == 0
    assert lib.numrs_hip_unary_forward(c.handle, L.GELU, pre2.ptr, y2.ptr, T * fout, 0.0) == 0
    assert np.array_equal(pre.numpy(), pre2.numpy()), "pre-activation"
    assert np.array_equal(y.numpy(), y2.numpy()), "fused forward != linear + gelu"
    ref_pre = O.matmul_f64(x, O.transpose(W)).astype(np.float64) + b
    assert_contraction(pre.numpy(), ref_pre, fin, what="pre")
    assert_close(y.numpy(), O.gelu(pre.numpy().astype(np.float64)), abs_tol=1e-6, rel_tol=1e-5,
                 what="y = gelu(pre)")
    prev = {k: rand(rng, s) for k, s in (("dx", (T, fin)), ("dW", (fout, fin)), ("db", fout))}
    gp = c.empty((T, fout))
    assert lib.numrs_hip_unary_backward(c.handle, L.GELU, gd.ptr, pre.ptr, gp.ptr, T * fout, 0.0,
                                        0) == 0
    for acc in ((0, 0, 0), (1, 0, 1)):
        dx, dW, db = (c.to_device(prev[k]) for k in ("dx", "dW", "db"))
        assert lib.numrs_hip_linear_gelu_backward(c.handle, gd.ptr, pre.ptr, xd.ptr, Wd.ptr, dx.ptr,
                                                  dW.ptr, db.ptr, T, fin, fout, *acc,
                                                  L.UNBROADCAST_CORRECT) == 0
        dx2, dW2, db2 = (c.to_device(prev[k]) for k in ("dx", "dW", "db"))
        assert lib.numrs_hip_linear_backward(c.handle, gp.ptr, xd.ptr, Wd.ptr, dx2.ptr, dW2.ptr,
                                             db2.ptr, T, fin, fout, *acc,
                                             L.UNBROADCAST_CORRECT) == 0
        for name, a, b2 in (("dx", dx, dx2), ("dW", dW, dW2), ("db", db, db2)):
            assert np.array_equal(a.numpy(), b2.numpy()), f"{name} {acc}: fused != composition"


# Cross-entropy loss forward: one workgroup for B <= 512 rows, the row kernel
# and a two-pass mean above.
@pytest.mark.parametrize("B,C", [(64, 10), (512, 33), (513, 10), (4096, 100)])
@pytest.mark.parametrize("labels_api", [False, True])
def test_cross_entropy_loss_forward(hip_ctx, rng, B, C, labels_api):
    say(f"ce loss B={B} C={C} labels={labels_api}")
    x = rand(rng, (B, C)) * 3
    lab = rng.integers(0, C, B).astype(np.int32)
    onehot = np.eye(C, dtype=np.float32)[lab]
    c = hip_ctx
    xd, out = c.to_device(x), c.empty((1,))
    if labels_api:
        ld = c.to_device(lab)
        rc = L.load().numrs_hip_cross_entropy_loss(c.handle, xd.ptr, None, ld.ptr, B, C, out.ptr)
    else:
        od = c.to_device(onehot)
        rc = L.load().numrs_hip_cross_entropy_loss(c.handle, xd.ptr, od.ptr, None, B, C, out.ptr)
    assert rc == 0
    x64 = x.astype(np.float64)
    m = x64.max(1, keepdims=True)
    lse = np.log(np.exp(x64 - m).sum(1)) + m[:, 0]
    ref = float((lse - x64[np.arange(B), lab]).mean())
    assert abs(float(out.numpy()[0]) - ref) <= 1e-5 + 1e-5 * abs(ref)
    assert abs(float(O.cross_entropy_loss(x, onehot)) - ref) <= 1e-5 + 1e-5 * abs(ref)


def test_optimizer_multi_tensor_bit_exact(hip_ctx, rng):
    import ctypes

    # (1 << 23) + 5 takes the float4 streaming body inside the multi-tensor launch
    sizes = [100352, 128, 1280, 10, 1, 4097, 33, (1 << 23) + 5]
    c = hip_ctx
    for kind in ("sgd", "sgd_mom", "adam"):
        ps = [rand(rng, n) for n in sizes]
        gs = [rand(rng, n) for n in sizes]
        ms = [np.zeros(n, np.float32) for n in sizes]
        vs = [np.zeros(n, np.float32) for n in sizes]
        pd = [c.to_device(a) for a in ps]
        gd = [c.to_device(a) for a in gs]
        md = [c.to_device(a) for a in ms]
        vd = [c.to_device(a) for a in vs]
        arr = lambda ds: (ctypes.c_void_p * len(ds))(*[d.ptr for d in ds])
        ns = (ctypes.c_int64 * len(sizes))(*sizes)
        for t in (1, 2, 3):
            if kind == "adam":
                rc = L.load().numrs_hip_adam_step_multi(c.handle, arr(pd), arr(gd), arr(md),
                                                        arr(vd), ns, len(sizes), 1e-3, 0.9, 0.999,
                                                        1e-8, 0.01, t)
                for i in range(len(sizes)):
                    O.adam_step(ps[i], gs[i], ms[i], vs[i], t, wd=0.01)
            else:
                mu = 0.9 if kind == "sgd_mom" else 0.0
                rc = L.load().numrs_hip_sgd_step_multi(c.handle, arr(pd), arr(gd),
                                                       arr(md) if mu else None, ns, len(sizes),
                                                       0.01, mu, 1e-4)
                for i in range(len(sizes)):
                    O.sgd_step(ps[i], gs[i], ms[i] if mu else None, 0.01, mu, 1e-4)
            assert rc == 0
        for i in range(len(sizes)):
            assert_bits(pd[i].numpy(), ps[i], f"{kind} p[{i}]")
