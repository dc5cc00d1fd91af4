"""Device context and device arrays over the C ABI (libnumrs_hip.so).

`Context` owns one numrs_hip_ctx (a HIP stream plus workspace) and exposes the
backward kernels with numpy-shaped arguments; `DeviceArray` is a device buffer
with a shape.  Every call checks the C status and raises `HipError` with the
library's message.
"""
from __future__ import annotations

import ctypes
from typing import Sequence

import numpy as np

from . import _lib as L


class HipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


class DeviceArray:
    """A device allocation holding a contiguous fp32/int32 array."""

    __slots__ = ("ctx", "ptr", "shape", "dtype", "_owned", "_base")

    def __init__(self, ctx: "Context", ptr: int, shape, dtype=np.float32, owned=True, base=None):
        self.ctx = ctx
        self.ptr = ptr
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self._owned = owned
        self._base = base  # the allocation a view keeps alive

    @property
    def size(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64))

    @property
    def nbytes(self) -> int:
        return self.size * self.dtype.itemsize

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if out.size:
            self.ctx._check(L.load().numrs_hip_download(self.ctx.handle, out.ctypes.data,
                                                        self.ptr, out.nbytes))
        return out

    def upload(self, host: np.ndarray) -> "DeviceArray":
        host = np.ascontiguousarray(host, dtype=self.dtype)
        if host.size != self.size:
            raise ValueError(f"upload of {host.shape} into {self.shape}")
        if host.size:
            self.ctx._check(L.load().numrs_hip_upload(self.ctx.handle, self.ptr, host.ctypes.data,
                                                      host.nbytes))
        return self

    def fill(self, value: float) -> "DeviceArray":
        self.ctx._check(L.load().numrs_hip_fill(self.ctx.handle, self.ptr, self.size, value))
        return self

    def view(self, offset_elems: int, shape) -> "DeviceArray":
        """A view starting `offset_elems` elements in; it holds a reference to
        the owning array, so the allocation lives as long as any view of it."""
        n = int(np.prod(tuple(int(s) for s in shape), dtype=np.int64))
        if offset_elems < 0 or offset_elems + n > self.size:
            raise ValueError(f"view of {n} elements at {offset_elems} outside {self.size}")
        base = self if self._owned else self._base
        return DeviceArray(self.ctx, self.ptr + offset_elems * self.dtype.itemsize, shape,
                           self.dtype, owned=False, base=base)

    def free(self) -> None:
        if self._owned and self.ptr and self.ctx.handle:
            L.load().numrs_hip_free(self.ctx.handle, self.ptr)
        self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _p(a) -> int | None:
    if a is None:
        return None
    return a.ptr


class Context:
    """One HIP stream on one gfx950 device (numrs_hip_create)."""

    def __init__(self, device: int = 0):
        lib = L.load()
        h = ctypes.c_void_p()
        rc = lib.numrs_hip_create(device, ctypes.byref(h))
        if rc != 0:
            raise HipError(rc, lib.numrs_hip_create_error().decode())
        self.handle = h.value
        self.device = device

    # -- plumbing -----------------------------------------------------------------
    def _check(self, rc: int) -> None:
        if rc != 0:
            raise HipError(rc, L.load().numrs_hip_last_error(self.handle).decode())

    def close(self) -> None:
        if self.handle:
            L.load().numrs_hip_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def info(self) -> tuple[int, str]:
        n = ctypes.c_int()
        buf = ctypes.create_string_buffer(64)
        self._check(L.load().numrs_hip_device_info(self.handle, ctypes.byref(n), buf, 64))
        return n.value, buf.value.decode()

    def empty(self, shape, dtype=np.float32) -> DeviceArray:
        shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        nbytes = int(np.prod(shape, dtype=np.int64)) * np.dtype(dtype).itemsize
        ptr = ctypes.c_void_p()
        self._check(L.load().numrs_hip_malloc(self.handle, nbytes, ctypes.byref(ptr)))
        return DeviceArray(self, ptr.value or 0, shape, dtype)

    def zeros(self, shape, dtype=np.float32) -> DeviceArray:
        a = self.empty(shape, dtype)
        if a.size:
            if np.dtype(dtype) == np.float32:
                a.fill(0.0)
            else:
                a.upload(np.zeros(a.shape, dtype))
        return a

    def to_device(self, host) -> DeviceArray:
        host = np.asarray(host)
        dtype = np.int32 if host.dtype.kind in "iu" else np.float32
        host = np.ascontiguousarray(host, dtype=dtype)
        return self.empty(host.shape, dtype).upload(host)

    def copy(self, dst: DeviceArray, src: DeviceArray, nbytes: int | None = None) -> None:
        """Device-to-device copy of nbytes (default: all of src) on the stream."""
        n = src.nbytes if nbytes is None else int(nbytes)
        if n > min(src.nbytes, dst.nbytes):
            raise ValueError("copy larger than an operand")
        self._check(L.load().numrs_hip_copy(self.handle, dst.ptr, src.ptr, n))

    def sync(self) -> None:
        self._check(L.load().numrs_hip_sync(self.handle))

    def reserve(self, nbytes: int) -> None:
        self._check(L.load().numrs_hip_reserve(self.handle, nbytes))

    def set_recurrence_mode(self, mode: str) -> None:
        """'auto' (persistent LSTM recurrences, ordinary launch, where they
        apply), 'per_step' (one launch per diagonal step), 'plain_launch'
        (the same as 'auto') or 'cooperative' (the persistent kernels through
        a cooperative launch).  Every mode gives the same bits."""
        code = {"auto": 0, "per_step": 1, "plain_launch": 2, "cooperative": 3}[mode]
        self._check(L.load().numrs_hip_set_recurrence_mode(self.handle, code))

    def set_split_reduction(self, mode: str) -> None:
        """'fused' (the default: split-K partials added inside the products'
        own launch) or 'separate' (one more launch after the products).  Both
        give the same bits."""
        code = {"fused": 0, "separate": 1}[mode]
        self._check(L.load().numrs_hip_set_split_reduction(self.handle, code))

    def set_persistent_wait_limit(self, rounds: int) -> None:
        """Poll rounds before a persistent kernel's wait gives up (negative:
        the default); a tiny limit forces the give-up path, for testing."""
        self._check(L.load().numrs_hip_set_persistent_wait_limit(self.handle, int(rounds)))

    def persistent_launches(self) -> int:
        """Persistent recurrence launches queued on this context so far."""
        return int(L.load().numrs_hip_persistent_launches(self.handle))

    def stream(self) -> int:
        return L.load().numrs_hip_stream(self.handle)

    def timer_record(self, slot: int) -> None:
        self._check(L.load().numrs_hip_timer_record(self.handle, slot))

    def timer_elapsed_ms(self, s0: int, s1: int) -> float:
        ms = ctypes.c_float()
        self._check(L.load().numrs_hip_timer_elapsed_ms(self.handle, s0, s1, ctypes.byref(ms)))
        return ms.value

    # -- contractions ---------------------------------------------------------------
    def matmul_backward(self, dC, A, B, dA=None, dB=None, accumulate=False) -> None:
        M, K = A.shape if A is not None else (dC.shape[0], B.shape[0])
        N = dC.shape[1]
        self._check(L.load().numrs_hip_matmul_backward(
            self.handle, _p(dC), _p(A), _p(B), _p(dA), _p(dB), M, K, N, int(accumulate)))

    def matmul_backward_batched(self, dC, A, B, dA=None, dB=None, accumulate=False) -> None:
        batch, M, K = A.shape
        N = dC.shape[2]
        self._check(L.load().numrs_hip_matmul_backward_batched(
            self.handle, _p(dC), _p(A), _p(B), _p(dA), _p(dB), batch, M, K, N, M * K, K * N,
            M * N, int(accumulate)))

    def matmul(self, A, B, C, trans_a=False, trans_b=False, accumulate=False) -> None:
        M = A.shape[1] if trans_a else A.shape[0]
        K = A.shape[0] if trans_a else A.shape[1]
        N = B.shape[0] if trans_b else B.shape[1]
        self._check(L.load().numrs_hip_matmul(self.handle, _p(A), _p(B), _p(C), M, K, N,
                                              int(trans_a), int(trans_b), int(accumulate)))

    def matmul_batched(self, A, B, C, trans_a=False, trans_b=False, accumulate=False) -> None:
        batch = A.shape[0]
        M = A.shape[2] if trans_a else A.shape[1]
        K = A.shape[1] if trans_a else A.shape[2]
        N = B.shape[1] if trans_b else B.shape[2]
        self._check(L.load().numrs_hip_matmul_batched(
            self.handle, _p(A), _p(B), _p(C), batch, M, K, N, M * K, K * N, M * N,
            int(trans_a), int(trans_b), int(accumulate)))

    # -- DispatchTable forward kernels (backend/dispatch.rs:51-93) -----------------------
    def elementwise(self, kind: int, a, b, out) -> None:
        """DispatchTable.elementwise: out = kind(a, b), same shapes; b unused by unary kinds."""
        self._check(L.load().numrs_hip_elementwise(self.handle, kind, _p(a), _p(b), _p(out),
                                                   a.size))

    def reduction(self, kind: int, x, axis: int | None, out) -> None:
        """DispatchTable.reduction over all elements (axis None) or one axis."""
        shp = (ctypes.c_int64 * max(len(x.shape), 1))(*x.shape)
        self._check(L.load().numrs_hip_reduction(self.handle, kind, _p(x), shp, len(x.shape),
                                                 -1 if axis is None else int(axis), _p(out)))

    # -- reductions ---------------------------------------------------------------------
    def sum_to_shape(self, g, out, mode=L.UNBROADCAST_CORRECT, accumulate=False) -> None:
        gs = (ctypes.c_int64 * max(len(g.shape), 1))(*g.shape)
        os_ = (ctypes.c_int64 * max(len(out.shape), 1))(*out.shape)
        self._check(L.load().numrs_hip_sum_to_shape(self.handle, _p(g), gs, len(g.shape), _p(out),
                                                    os_, len(out.shape), mode, int(accumulate)))

    def relu_bias_backward(self, g, z, dx=None, db=None, mode=L.UNBROADCAST_CORRECT,
                           accumulate=False) -> None:
        rows, cols = g.shape
        self._check(L.load().numrs_hip_relu_bias_backward(
            self.handle, _p(g), _p(z), _p(dx), _p(db), rows, cols, mode, int(accumulate)))

    # -- elementwise ---------------------------------------------------------------------
    def unary_backward(self, kind: int, g, v, dx, param: float = 0.0, accumulate=False) -> None:
        self._check(L.load().numrs_hip_unary_backward(self.handle, kind, _p(g), _p(v), _p(dx),
                                                      g.size, param, int(accumulate)))

    def binary_backward(self, kind: int, g, x, y, dx, dy, accumulate=False) -> None:
        self._check(L.load().numrs_hip_binary_backward(self.handle, kind, _p(g), _p(x), _p(y),
                                                       _p(dx), _p(dy), g.size, int(accumulate)))

    def fill_grad(self, g_scalar, dx, divide_by_n=False, accumulate=False) -> None:
        self._check(L.load().numrs_hip_fill_grad(self.handle, _p(g_scalar), _p(dx), dx.size,
                                                 int(divide_by_n), int(accumulate)))

    def mse_backward(self, g_scalar, p, t, dp, dt=None, accumulate=False) -> None:
        self._check(L.load().numrs_hip_mse_backward(self.handle, _p(g_scalar), _p(p), _p(t),
                                                    _p(dp), _p(dt), p.size, int(accumulate)))

    # -- row-wise ---------------------------------------------------------------------------
    def softmax_ce_backward(self, g_scalar, logits, dlogits, onehot=None, labels=None,
                            accumulate=False) -> None:
        B, C = logits.shape
        self._check(L.load().numrs_hip_softmax_ce_backward(
            self.handle, _p(g_scalar), _p(logits), _p(onehot), _p(labels), _p(dlogits), B, C,
            int(accumulate)))

    def softmax_backward(self, y, g, dx, accumulate=False) -> None:
        rows, cols = y.shape[0], int(np.prod(y.shape[1:]))
        self._check(L.load().numrs_hip_softmax_backward(self.handle, _p(y), _p(g), _p(dx), rows,
                                                        cols, int(accumulate)))

    def argmax_rows(self, x, idx, tie_last=False) -> None:
        rows, cols = x.shape
        self._check(L.load().numrs_hip_argmax_rows(self.handle, _p(x), _p(idx), rows, cols,
                                                   int(tie_last)))

    # -- optimizers -------------------------------------------------------------------------
    def sgd_step(self, p, g, v=None, lr=0.01, mu=0.0, wd=0.0) -> None:
        self._check(L.load().numrs_hip_sgd_step(self.handle, _p(p), _p(g), _p(v), p.size, lr,
                                                mu, wd))

    def adam_step(self, p, g, m, v, t: int, lr=1e-3, b1=0.9, b2=0.999, eps=1e-8,
                  wd=0.0) -> None:
        self._check(L.load().numrs_hip_adam_step(self.handle, _p(p), _p(g), _p(m), _p(v), p.size,
                                                 lr, b1, b2, eps, wd, int(t)))

    def optimizer_step(self, kind: int, ps, gs, s1s, s2s, hyper, t: int = 0) -> None:
        """numrs_hip_optimizer_step over lists of device arrays (None = no slot)."""
        k = len(ps)

        def arr(xs):
            if xs is None:
                return None
            return (ctypes.c_void_p * max(k, 1))(*[_p(x) for x in xs])

        n = (ctypes.c_int64 * max(k, 1))(*[x.size for x in ps])
        h = (ctypes.c_float * len(hyper))(*[float(x) for x in hyper])
        self._check(L.load().numrs_hip_optimizer_step(
            self.handle, kind, arr(ps), arr(gs), arr(s1s), arr(s2s), n, k, h, len(hyper), int(t)))

    def lookahead_update(self, fast, slow, alpha: float) -> None:
        k = len(fast)
        fa = (ctypes.c_void_p * max(k, 1))(*[_p(x) for x in fast])
        sa = (ctypes.c_void_p * max(k, 1))(*[_p(x) for x in slow])
        n = (ctypes.c_int64 * max(k, 1))(*[x.size for x in fast])
        self._check(L.load().numrs_hip_lookahead_update(self.handle, fa, sa, n, k, alpha))

    def dot(self, x, y, out) -> None:
        self._check(L.load().numrs_hip_dot(self.handle, _p(x), _p(y), x.size, _p(out)))


def shape_of(x: Sequence[int] | DeviceArray) -> tuple[int, ...]:
    return x.shape if isinstance(x, DeviceArray) else tuple(x)
