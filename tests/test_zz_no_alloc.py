"""The allocation-free fused ReLU + bias backward
(numrs_hip_relu_bias_backward_noalloc) against the allocating entry point
numrs_hip_relu_bias_backward, through the C ABI, on the GPU.

The two share their kernels; only where the column-sum partials live differs
(a static per-GPU array instead of the context workspace), so results must
be identical bit for bit.  Two calls in a row, the second with a smaller
input, check that the array's leftover contents from the first call do not
leak into the second.
"""
import numpy as np
import pytest

from numrs_amd import _lib as L
from oracle import oracle as O
from tests.conftest import assert_bits, assert_sum, rand

pytestmark = pytest.mark.gpu

NOALLOC = "numrs_hip_relu_bias_backward_noalloc"
ALLOC = "numrs_hip_relu_bias_backward"


def _call(c, fn, g, z, dx, db, mode, acc):
    rows, cols = g.shape
    return getattr(L.load(), fn)(c.handle, g.ptr, z.ptr, dx.ptr if dx is not None else None,
                                 db.ptr if db is not None else None, rows, cols, mode, acc)


@pytest.mark.parametrize("mode", [L.UNBROADCAST_CORRECT, L.UNBROADCAST_REFERENCE])
@pytest.mark.parametrize("acc", [0, 1])
def test_noalloc_matches_allocating_entry(hip_ctx, mode, acc):
    c = hip_ctx
    rng = np.random.default_rng(7000 + 10 * mode + acc)
    # The C3 shape, then a smaller ragged one on the same array.
    for rows, cols in ((4096, 4096), (300, 1001)):
        print(f"[gpu] noalloc relu+bias {rows}x{cols} mode={mode} acc={acc}", flush=True)
        g, z = rand(rng, (rows, cols)), rand(rng, (rows, cols))
        dx0, db0 = rand(rng, (rows, cols)), rand(rng, cols)
        gd, zd = c.to_device(g), c.to_device(z)
        dx_a, db_a = c.to_device(dx0), c.to_device(db0)
        dx_n, db_n = c.to_device(dx0), c.to_device(db0)
        assert _call(c, ALLOC, gd, zd, dx_a, db_a, mode, acc) == 0
        assert _call(c, NOALLOC, gd, zd, dx_n, db_n, mode, acc) == 0, \
            L.load().numrs_hip_last_error(c.handle)
        assert_bits(dx_n.numpy(), dx_a.numpy(), "dx: noalloc vs allocating")
        assert_bits(db_n.numpy(), db_a.numpy(), "db: noalloc vs allocating")
        # and against the oracle (relu_backward, backward.rs:152-163)
        rdx = O.relu_backward(g, z)
        assert_bits(dx_n.numpy(), rdx + dx0 if acc else rdx, "dx vs oracle")
        if mode == L.UNBROADCAST_CORRECT:
            ref = rdx.astype(np.float64).sum(0) + (db0 if acc else 0)
            assert_sum(db_n.numpy(), ref, rows, what="db vs float64")


def test_noalloc_dx_only_and_empty(hip_ctx):
    c = hip_ctx
    rng = np.random.default_rng(7100)
    g, z = rand(rng, (64, 96)), rand(rng, (64, 96))
    dx = c.empty((64, 96))
    assert _call(c, NOALLOC, c.to_device(g), c.to_device(z), dx, None,
                 L.UNBROADCAST_CORRECT, 0) == 0
    assert_bits(dx.numpy(), O.relu_backward(g, z), "dx only")
    # zero rows: db is the empty sum
    e = c.zeros(8).view(0, (0, 8))
    db = c.to_device(np.full(8, 3.0, np.float32))
    assert _call(c, NOALLOC, e, e, None, db, L.UNBROADCAST_CORRECT, 0) == 0
    assert (db.numpy() == 0).all()


def test_noalloc_rejects_partials_beyond_the_array(hip_ctx):
    c = hip_ctx
    cols = (1 << 20) + 4
    g = c.zeros(cols).view(0, (1, cols))
    db = c.zeros(cols)
    rc = _call(c, NOALLOC, g, g, None, db, L.UNBROADCAST_CORRECT, 0)
    assert rc == L.E_INVALID
    assert b"allocation-free" in L.load().numrs_hip_last_error(c.handle)
