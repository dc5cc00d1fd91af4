"""CPU-side checks of the C ABI: the library loads, exports every function the
header declares, and its host-side argument checks fail loudly (no GPU work)."""
import ctypes
import os

import pytest

import numrs_amd
from numrs_amd import _lib as L


def test_library_built_in_tree():
    assert os.path.exists(L.LIB_PATH), "run python -m numrs_amd.build"
    assert os.path.dirname(L.LIB_PATH).endswith(os.path.join("numrs_amd", "lib"))


def test_exports_every_header_function():
    lib = L.load()
    names = L.header_functions()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared in numrs_hip.h but not exported: {missing}"
    undeclared = sorted(set(L.SIGNATURES) - set(names))
    assert not undeclared, f"bound in _lib.py but not in the header: {undeclared}"
    unbound = sorted(set(names) - set(L.SIGNATURES))
    assert not unbound, f"declared but not bound by ctypes: {unbound}"


def test_null_context_is_rejected():
    lib = L.load()
    assert lib.numrs_hip_sync(None) == L.E_INVALID
    assert lib.numrs_hip_matmul_backward(None, None, None, None, None, None, 1, 1, 1, 0) == L.E_INVALID
    assert lib.numrs_hip_last_error(None) == b"null context"


def test_create_rejects_missing_device_without_gpu():
    # In the CPU container there is no GPU: creation must fail with a message,
    # never fall back to a host path.
    import torch

    if torch.cuda.device_count() > 0:
        pytest.skip("a GPU is present")
    lib = L.load()
    h = ctypes.c_void_p()
    rc = lib.numrs_hip_create(0, ctypes.byref(h))
    assert rc == L.E_NODEV
    assert h.value is None
    assert lib.numrs_hip_create_error()
    with pytest.raises(numrs_amd.HipError):
        numrs_amd.Context(0)


def test_header_enums_match_bindings():
    text = open(L.HEADER_PATH).read()
    for name, val in [("NUMRS_HIP_RELU", L.RELU), ("NUMRS_HIP_POW", L.POW),
                      ("NUMRS_HIP_DIV", L.DIV), ("NUMRS_HIP_UNBROADCAST_REFERENCE",
                                                 L.UNBROADCAST_REFERENCE),
                      ("NUMRS_HIP_E_NODEV", L.E_NODEV)]:
        assert f"{name} = {val}" in text, name


def test_grad_mode_is_thread_local_host_state():
    # autograd/mod.rs:194-206: is_grad_enabled / set_grad_enabled, no GPU involved
    import threading

    from numrs_amd import is_grad_enabled, no_grad, set_grad_enabled

    assert is_grad_enabled()
    with no_grad():
        assert not is_grad_enabled()
        seen = []
        t = threading.Thread(target=lambda: seen.append(is_grad_enabled()))
        t.start()
        t.join()
        assert seen == [True]
    assert is_grad_enabled()
    set_grad_enabled(False)
    set_grad_enabled(True)
    assert is_grad_enabled()
