import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


# Gradient tolerance of the north star: |g - r| <= ABS + REL * |r| (fp32).
ABS_TOL = 1e-5
REL_TOL = 1e-4


def assert_close(got, ref, abs_tol=ABS_TOL, rel_tol=REL_TOL, what=""):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} vs {ref.shape}"
    err = np.abs(got - ref)
    bound = abs_tol + rel_tol * np.abs(ref)
    bad = ~(err <= bound)
    if bad.any():
        i = np.flatnonzero(bad.ravel())[0]
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{bad.size} outside |g-r| <= {abs_tol} + {rel_tol}|r|; "
            f"first at flat {i}: got {got.ravel()[i]!r} ref {ref.ravel()[i]!r}; "
            f"max err {err.max():.3e}")


U32 = 2.0 ** -24  # fp32 unit roundoff


def contraction_allowance(K, rms_ab=1.0):
    """fp32 rounding allowance of a length-K sum of products with rms(a*b) =
    rms_ab: partial sums grow like sqrt(K)*rms_ab over K roundings, so the
    error scale is u*K*rms_ab; 4x that bounds numrs's own sequential fp32
    loop (backward.rs:123-146) at K = 2048 and 4096."""
    return 4.0 * U32 * K * rms_ab


def assert_contraction(got, ref64, K, rms_ab=1.0, ref32=None, what=""):
    """A gradient produced by a length-K fp32 contraction (matmul grads),
    against the float64-accumulated oracle.

    Per element: |g - r| <= 1e-5 + 1e-4|r| + contraction_allowance(K): the
    north-star tolerance plus the fp32 rounding allowance that the
    reference's own fp32 result also needs (tests/test_oracle.py::
    test_reference_fp32_needs_contraction_allowance shows it misses the bare
    bound at K = 2048).
    Aggregate, when the reference's fp32 result `ref32` is given: the mean
    error must be no more than 0.8x the reference's own mean error, i.e. the
    GPU result is at least as close to the exact gradient as numrs's CPU one."""
    assert_close(got, ref64, abs_tol=ABS_TOL + contraction_allowance(K, rms_ab), what=what)
    if ref32 is not None:
        g = np.asarray(got, np.float64)
        r = np.asarray(ref64, np.float64)
        e_gpu = np.abs(g - r).mean()
        e_ref = np.abs(np.asarray(ref32, np.float64) - r).mean()
        assert e_gpu <= 0.8 * e_ref + 1e-7, (
            f"{what}: mean error {e_gpu:.3e} vs numrs fp32 loop {e_ref:.3e}")


def assert_sum(got, ref64, n, ref32=None, what=""):
    """A result produced by length-n fp32 sums (column sums, bias grads),
    against the float64 sum.

    Per element: |g - r| <= 1e-5 + 1e-4|r| + 2e-7 n.  A column whose terms
    cancel to near zero keeps the rounding of its partial sums, which no fp32
    order avoids (on a 4096 x 2048 N(0,1) matrix numrs's own sequential loop
    misses the bare bound on 4 columns, by up to 1.4x); 2e-7 n is the
    allowance the axis-reduction tests use.
    Aggregate, when numrs's sequential fp32 result `ref32` is given: the mean
    error must be at most 0.8x that loop's mean error."""
    assert_close(got, ref64, abs_tol=ABS_TOL + 2e-7 * n, what=what)
    if ref32 is not None:
        r = np.asarray(ref64, np.float64)
        e_gpu = np.abs(np.asarray(got, np.float64) - r).mean()
        e_ref = np.abs(np.asarray(ref32, np.float64) - r).mean()
        assert e_gpu <= 0.8 * e_ref + 1e-7, (
            f"{what}: mean error {e_gpu:.3e} vs numrs sequential fp32 sum {e_ref:.3e}")


def assert_chain(got, ref64, cpu32, what="", mean_factor=1.0, max_factor=1.5, factor_min_size=1):
    """A gradient at the end of a long fp32 chain (the C4 block, the C5 BPTT),
    against the float64 oracle `ref64` and the same chain run in fp32 on the
    CPU (`cpu32`, numpy float32 through the same oracle).

    Per element, the north-star bound |g - r| <= 1e-5 + 1e-4|r|, and the same
    bound with its absolute term scaled to the tensor, 1e-5 * max|r| (the MSE
    over millions of outputs makes these grads 1e-4..1e-10, where a fixed
    1e-5 would accept anything).
    Per tensor: the mean error at most `mean_factor` times the fp32 CPU
    chain's (1: no larger) and the largest error at most `max_factor` times
    its largest, for tensors of at least `factor_min_size` elements (on a
    handful of elements these ratios compare two rounding patterns by
    chance); and the norm-wise relative error below 2e-6."""
    g = np.asarray(got, np.float64)
    r = np.asarray(ref64, np.float64)
    c = np.asarray(cpu32, np.float64)
    assert_close(g, r, what=what)
    assert_close(g, r, abs_tol=1e-5 * np.abs(r).max(), what=f"{what} (scaled abs term)")
    eg, ec = np.abs(g - r), np.abs(c - r)
    if g.size < factor_min_size:
        mean_factor = max_factor = np.inf
    assert eg.mean() <= mean_factor * ec.mean() + 1e-300, (
        f"{what}: mean error {eg.mean():.3e} above {mean_factor}x the fp32 CPU chain's "
        f"{ec.mean():.3e}")
    assert eg.max() <= max_factor * ec.max() + 1e-300, (
        f"{what}: max error {eg.max():.3e} above {max_factor}x the fp32 CPU chain's {ec.max():.3e}")
    nrel = np.linalg.norm(g - r) / max(np.linalg.norm(r), 1e-300)
    assert nrel < 2e-6, f"{what}: norm-relative error {nrel:.3e}"


def seq_colsum32(x):
    """Column sums of a 2-D fp32 array in numrs's order: one sequential fp32
    accumulation down each column (add.accumulate is sequential)."""
    x = np.asarray(x, np.float32)
    if x.shape[0] == 0:
        return np.zeros(x.shape[1], np.float32)
    return np.add.accumulate(x, axis=0, dtype=np.float32)[-1]


def assert_bits(got, ref, what=""):
    got = np.ascontiguousarray(got, np.float32)
    ref = np.ascontiguousarray(ref, np.float32)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} vs {ref.shape}"
    gb, rb = got.view(np.uint32), ref.view(np.uint32)
    # Treat every NaN payload as equal.
    same = (gb == rb) | (np.isnan(got) & np.isnan(ref))
    if not same.all():
        i = np.flatnonzero(~same.ravel())[0]
        raise AssertionError(f"{what}: {int((~same).sum())} elements differ in bits; first at {i}: "
                             f"got {got.ravel()[i]!r} ref {ref.ravel()[i]!r}")


@pytest.fixture(scope="session")
def hip_ctx():
    """One HIP context for the whole GPU session (fails loudly without the library)."""
    from numrs_amd import Context
    ctx = Context(0)
    yield ctx
    ctx.close()


def rand(rng, shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float32)
