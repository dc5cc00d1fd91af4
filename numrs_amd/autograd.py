"""numrs's autograd Tensor on the GPU (mirrors numrs-core/src/autograd).

`Tensor` wraps a numrs_hip_tensor handle of the C ABI: values and grads stay in
device memory, every op records a node when grad mode is on, and
`backward()` runs the whole reverse sweep as kernels on the context's stream.
Names and argument meaning follow the reference's Rust API
(autograd/tensor.rs, autograd/ops.rs): `Tensor.new(data, requires_grad)`,
`a.matmul(b)`, `c.backward()`, `a.gradient()` (None when the tensor has no
grad), `values()`, `shape()`, `item()`, `zero_grad()`, `detach()`.
"""
from __future__ import annotations

import contextlib
import ctypes
import threading

import numpy as np

from . import _lib as L
from .device import Context, HipError

_default = threading.local()


def default_context() -> Context:
    """The calling thread's context on device 0 (created on first use)."""
    ctx = getattr(_default, "ctx", None)
    if ctx is None:
        ctx = Context(0)
        _default.ctx = ctx
    return ctx


def set_default_context(ctx: Context) -> None:
    _default.ctx = ctx


def is_grad_enabled() -> bool:
    """autograd/mod.rs:199-201 (thread-local)."""
    return bool(L.load().numrs_hip_is_grad_enabled())


def set_grad_enabled(enabled: bool) -> None:
    """autograd/mod.rs:204-206."""
    L.load().numrs_hip_set_grad_enabled(int(bool(enabled)))


@contextlib.contextmanager
def no_grad():
    """NoGrad guard / no_grad! macro (autograd/mod.rs:209-246)."""
    prev = is_grad_enabled()
    set_grad_enabled(False)
    try:
        yield
    finally:
        set_grad_enabled(prev)


def set_unbroadcast_mode(mode: str, ctx: Context | None = None) -> None:
    """'correct' (axis sums, default) or 'reference' (numrs's full sum into
    element 0, backward.rs:12-39 + tensor.rs:120-132) for broadcast grads."""
    ctx = ctx or default_context()
    code = {"correct": L.UNBROADCAST_CORRECT, "reference": L.UNBROADCAST_REFERENCE}[mode]
    ctx._check(L.load().numrs_hip_set_unbroadcast_mode(ctx.handle, code))


def _shape_arr(shape):
    shape = tuple(int(s) for s in shape)
    return (ctypes.c_int64 * max(len(shape), 1))(*shape), len(shape)


class Tensor:
    """Device-resident autograd tensor (autograd/tensor.rs:18-33)."""

    __slots__ = ("_h", "ctx")

    def __init__(self, handle: int, ctx: Context):
        self._h = handle
        self.ctx = ctx

    # -- construction ------------------------------------------------------------
    @staticmethod
    def new(data, requires_grad: bool = False, shape=None, ctx: Context | None = None) -> "Tensor":
        """Tensor::new(Array::new(shape, data), requires_grad) (tensor.rs:41-59)."""
        ctx = ctx or default_context()
        arr = np.ascontiguousarray(np.asarray(data, dtype=np.float32))
        if shape is not None:
            arr = arr.reshape(shape)
        sa, nd = _shape_arr(arr.shape)
        h = ctypes.c_void_p()
        ctx._check(L.load().numrs_hip_tensor_new(ctx.handle, arr.ctypes.data if arr.size else None,
                                                 sa, nd, int(requires_grad), ctypes.byref(h)))
        return Tensor(h.value, ctx)

    def __del__(self):
        try:
            if self._h:
                L.load().numrs_hip_tensor_free(self._h)
                self._h = None
        except Exception:
            pass

    def _out(self, rc: int, h: ctypes.c_void_p) -> "Tensor":
        self.ctx._check(rc)
        return Tensor(h.value, self.ctx)

    # -- metadata / data ---------------------------------------------------------------
    def shape(self) -> tuple[int, ...]:
        buf = (ctypes.c_int64 * 8)()
        nd = L.load().numrs_hip_tensor_shape(self._h, buf, 8)
        return tuple(buf[i] for i in range(nd))

    @property
    def requires_grad(self) -> bool:
        return bool(L.load().numrs_hip_tensor_requires_grad(self._h))

    @property
    def is_leaf(self) -> bool:
        return bool(L.load().numrs_hip_tensor_is_leaf(self._h))

    def numel(self) -> int:
        return int(L.load().numrs_hip_tensor_numel(self._h))

    def values(self) -> np.ndarray:
        """Tensor::values (tensor.rs:91-93), as an array of the tensor's shape."""
        out = np.empty(self.shape(), np.float32)
        self.ctx._check(L.load().numrs_hip_tensor_values(self._h, out.ctypes.data, out.size))
        return out

    def item(self) -> float:
        """Tensor::item (tensor.rs:101-107)."""
        v = self.values().ravel()
        return float(v[0]) if v.size else 0.0

    def gradient(self) -> np.ndarray | None:
        """Tensor::gradient (tensor.rs:96-98): None when the tensor has no grad."""
        out = np.empty(self.shape(), np.float32)
        rc = L.load().numrs_hip_tensor_gradient(self._h, out.ctypes.data, out.size)
        if rc < 0:
            self.ctx._check(rc)
        return out if rc == 1 else None

    grad = gradient  # the bindings' name (numrs-c tensor.rs:53-67)

    def set_gradient(self, g) -> None:
        g = np.ascontiguousarray(g, np.float32)
        self.ctx._check(L.load().numrs_hip_tensor_set_gradient(self._h, g.ctypes.data, g.size))

    def zero_grad(self) -> None:
        self.ctx._check(L.load().numrs_hip_tensor_zero_grad(self._h))

    def device_ptrs(self) -> tuple[int, int | None]:
        d, g = ctypes.c_void_p(), ctypes.c_void_p()
        self.ctx._check(L.load().numrs_hip_tensor_device_ptrs(self._h, ctypes.byref(d),
                                                              ctypes.byref(g)))
        return d.value, g.value

    def backward(self) -> None:
        """Tensor::backward (tensor.rs:173-215)."""
        self.ctx._check(L.load().numrs_hip_tensor_backward(self._h))

    def detach(self) -> "Tensor":
        h = ctypes.c_void_p()
        return self._out(L.load().numrs_hip_tensor_detach(self._h, ctypes.byref(h)), h)

    # -- ops (autograd/ops.rs) -----------------------------------------------------------
    def _bin(self, kind: int, other: "Tensor") -> "Tensor":
        h = ctypes.c_void_p()
        return self._out(L.load().numrs_hip_tensor_binary(kind, self._h, other._h, ctypes.byref(h)), h)

    def add(self, other: "Tensor") -> "Tensor":
        return self._bin(L.ADD, other)

    def sub(self, other: "Tensor") -> "Tensor":
        return self._bin(L.SUB, other)

    def mul(self, other: "Tensor") -> "Tensor":
        return self._bin(L.MUL, other)

    def div(self, other: "Tensor") -> "Tensor":
        return self._bin(L.DIV, other)

    __add__, __sub__, __mul__, __truediv__ = add, sub, mul, div

    def __matmul__(self, other):
        return self.matmul(other)

    def _un(self, kind: int, param: float = 0.0) -> "Tensor":
        h = ctypes.c_void_p()
        return self._out(L.load().numrs_hip_tensor_unary(kind, self._h, param, ctypes.byref(h)), h)

    def relu(self):
        return self._un(L.RELU)

    def sigmoid(self):
        return self._un(L.SIGMOID)

    def tanh(self):
        return self._un(L.TANH)

    def exp(self):
        return self._un(L.EXP)

    def log(self):
        return self._un(L.LOG)

    def sqrt(self):
        return self._un(L.SQRT)

    def sin(self):
        return self._un(L.SIN)

    def cos(self):
        return self._un(L.COS)

    def tan(self):
        return self._un(L.TAN)

    def gelu(self):
        return self._un(L.GELU)

    def pow(self, exponent: float):
        return self._un(L.POW, float(exponent))

    def matmul(self, other: "Tensor") -> "Tensor":
        h = ctypes.c_void_p()
        return self._out(L.load().numrs_hip_tensor_matmul(self._h, other._h, ctypes.byref(h)), h)

    def transpose(self) -> "Tensor":
        h = ctypes.c_void_p()
        return self._out(L.load().numrs_hip_tensor_transpose(self._h, ctypes.byref(h)), h)

    def reshape(self, shape) -> "Tensor":
        """Tensor::reshape (ops.rs:353-369): a new tensor holding a copy of the
        values in `shape`; its backward reshapes the grad back
        (reshape_backward, backward.rs:324-330)."""
        sa, nd = _shape_arr(shape)
        h = ctypes.c_void_p()
        return self._out(L.load().numrs_hip_tensor_reshape(self._h, sa, nd, ctypes.byref(h)), h)

    def flatten(self, start_dim: int = 0, end_dim: int | None = None) -> "Tensor":
        """Tensor::flatten(start_dim, end_dim) (ops.rs:336-351, ops/shape/flatten.rs:13-43):
        dims start_dim..=end_dim merge into one; end_dim is clamped to the last
        dim.  The backward is flatten_backward (backward.rs:315-321)."""
        shape = self.shape()
        nd = len(shape)
        end = nd - 1 if end_dim is None or end_dim >= nd else int(end_dim)
        if start_dim > end:
            raise ValueError(f"flatten: start_dim ({start_dim}) cannot come after end_dim ({end})")
        flat = int(np.prod(shape[start_dim:end + 1], dtype=np.int64))
        return self.reshape(tuple(shape[:start_dim]) + (flat,) + tuple(shape[end + 1:]))

    def _axis(self, axis: int) -> int:
        nd = len(self.shape())
        a = axis + nd if axis < 0 else axis
        if not 0 <= a < nd:
            raise ValueError(f"axis {axis} out of range for {nd} dimensions")
        return a

    def sum(self, axis: int | None = None) -> "Tensor":
        """Tensor::sum (ops.rs:214-231): all elements into shape [1]; with an
        axis, that axis is removed (ops::sum(a, Some(axis)))."""
        h = ctypes.c_void_p()
        if axis is None:
            return self._out(L.load().numrs_hip_tensor_sum(self._h, 0, ctypes.byref(h)), h)
        return self._out(L.load().numrs_hip_tensor_sum_axis(self._h, self._axis(axis), 0,
                                                             ctypes.byref(h)), h)

    def mean(self, axis: int | None = None) -> "Tensor":
        """Tensor::mean (ops.rs:234-252); with an axis, ops::mean(a, Some(axis))."""
        h = ctypes.c_void_p()
        if axis is None:
            return self._out(L.load().numrs_hip_tensor_sum(self._h, 1, ctypes.byref(h)), h)
        return self._out(L.load().numrs_hip_tensor_sum_axis(self._h, self._axis(axis), 1,
                                                             ctypes.byref(h)), h)

    def mse_loss(self, target: "Tensor") -> "Tensor":
        h = ctypes.c_void_p()
        return self._out(L.load().numrs_hip_tensor_mse_loss(self._h, target._h, ctypes.byref(h)), h)

    def cross_entropy_loss(self, target: "Tensor") -> "Tensor":
        h = ctypes.c_void_p()
        return self._out(L.load().numrs_hip_tensor_cross_entropy_loss(self._h, target._h,
                                                                      ctypes.byref(h)), h)

    def cross_entropy_labels(self, labels) -> "Tensor":
        lab = np.ascontiguousarray(labels, np.int32)
        if lab.size != self.shape()[0]:
            raise ValueError("one label per row")
        h = ctypes.c_void_p()
        return self._out(L.load().numrs_hip_tensor_cross_entropy_labels(self._h, lab.ctypes.data,
                                                                        ctypes.byref(h)), h)

    def softmax(self, axis: int = -1) -> "Tensor":
        """Softmax along `axis` (default the last, row kernels); the reference
        rejects an axis (ops/stats/softmax.rs:13-16)."""
        h = ctypes.c_void_p()
        a = self._axis(axis)
        if a == len(self.shape()) - 1:
            return self._out(L.load().numrs_hip_tensor_softmax(self._h, ctypes.byref(h)), h)
        return self._out(L.load().numrs_hip_tensor_softmax_axis(self._h, a, ctypes.byref(h)), h)

    def layer_norm(self, gamma: "Tensor", beta: "Tensor", eps: float = 1e-5) -> "Tensor":
        h = ctypes.c_void_p()
        return self._out(L.load().numrs_hip_tensor_layer_norm(self._h, gamma._h, beta._h, eps,
                                                              ctypes.byref(h)), h)

    def linear(self, weight: "Tensor", bias: "Tensor | None" = None, relu: bool = False,
               residual: "Tensor | None" = None, gelu: bool = False) -> "Tensor":
        """self @ weight^T + bias as one node (Linear::forward's values and
        grads).  relu=True / gelu=True also apply that activation in the same
        node (the Linear -> ReLU / GELU pair); residual=r returns r + (self @
        weight^T + bias) as one node (the Linear then Add of a residual
        block).  Each gives the same values and gradients as the separate
        nodes."""
        h = ctypes.c_void_p()
        lib = L.load()
        b = bias._h if bias is not None else None
        if relu + gelu + (residual is not None) > 1:
            raise ValueError("linear: at most one of relu, gelu and residual")
        if residual is not None:
            return self._out(lib.numrs_hip_tensor_linear_residual(self._h, weight._h, b,
                                                                  residual._h, ctypes.byref(h)), h)
        fn = (lib.numrs_hip_tensor_linear_relu if relu else
              lib.numrs_hip_tensor_linear_gelu if gelu else lib.numrs_hip_tensor_linear)
        return self._out(fn(self._h, weight._h, b, ctypes.byref(h)), h)

    def lstm(self, w_ih: "Tensor", w_hh: "Tensor", bias: "Tensor | None" = None) -> "Tensor":
        """LSTM layer over self [B, T, I] -> hidden states [B, T, H]."""
        h = ctypes.c_void_p()
        return self._out(L.load().numrs_hip_tensor_lstm(self._h, w_ih._h, w_hh._h,
                                                        bias._h if bias is not None else None,
                                                        ctypes.byref(h)), h)

    def lstm2(self, w_ih1: "Tensor", w_hh1: "Tensor", b1: "Tensor | None", w_ih2: "Tensor",
              w_hh2: "Tensor", b2: "Tensor | None") -> "Tensor":
        """Two stacked LSTM layers over self [B, T, I] as one node -> the
        upper layer's hidden states [B, T, H2] (zero initial states)."""
        h = ctypes.c_void_p()
        opt = lambda t: t._h if t is not None else None
        return self._out(L.load().numrs_hip_tensor_lstm2(self._h, w_ih1._h, w_hh1._h, opt(b1),
                                                         w_ih2._h, w_hh2._h, opt(b2),
                                                         ctypes.byref(h)), h)

    def time_slice(self, t: int) -> "Tensor":
        """self[:, t, :] of a [B, T, D] tensor."""
        h = ctypes.c_void_p()
        return self._out(L.load().numrs_hip_tensor_time_slice(self._h, int(t), ctypes.byref(h)), h)

    def attention(self, k: "Tensor", v: "Tensor", batch: int, seq: int, heads: int) -> "Tensor":
        """Multi-head attention with self as q; q, k, v are [batch*seq, dim]."""
        h = ctypes.c_void_p()
        return self._out(L.load().numrs_hip_tensor_attention(self._h, k._h, v._h, batch, seq, heads,
                                                             ctypes.byref(h)), h)

    def attention_qkv(self, batch: int, seq: int, heads: int) -> "Tensor":
        """Multi-head attention over self = a packed projection [batch*seq, 3*dim]
        whose column blocks are q, k and v; returns [batch*seq, dim]."""
        h = ctypes.c_void_p()
        return self._out(L.load().numrs_hip_tensor_attention_qkv(self._h, batch, seq, heads,
                                                                 ctypes.byref(h)), h)

    def __repr__(self) -> str:
        return f"Tensor(shape={list(self.shape())}, requires_grad={self.requires_grad})"


__all__ = ["Tensor", "no_grad", "is_grad_enabled", "set_grad_enabled", "set_unbroadcast_mode",
           "default_context", "set_default_context", "HipError"]
