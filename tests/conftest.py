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
