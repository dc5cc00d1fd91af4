"""numpy-facing wrapper of the C oracle (oracle/numrs_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker.  The product library never
imports this module.  Every arithmetic function forwards to the C restatement,
which cites the numrs reference file:line it follows; the shape-only functions
(reshape / flatten) are restated here in Python with their citations.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "build", "liboracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_i = ctypes.c_int


def build() -> None:
    """Compile the oracle with its Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        _lib = ctypes.CDLL(_SO)
        _declare(_lib)
    return _lib


def _declare(L) -> None:
    sig = {
        "orc_sum_avx2_order": (_f32, [_f32p, _i64]),
        "orc_sum_seq": (_f32, [_f32p, _i64]),
        "orc_sum_rows_avx2_order": (None, [_f32p, _i64, _i64, _f32p]),
        "orc_sum_avx2_order_mt": (_f32, [_f32p, _i64, _i]),
        "orc_transpose": (None, [_f32p, _i64, _i64, _f32p]),
        "orc_accumulate": (None, [_f32p, _i64, _f32p, _i64]),
        "orc_matmul_backward_rows": (None, [_f32p] * 5 + [_i64] * 7),
        "orc_matmul_backward": (None, [_f32p] * 5 + [_i64] * 3),
        "orc_matmul_backward_f64_rows": (None, [_f32p] * 5 + [_i64] * 7 + [_f64p]),
        "orc_matmul_backward_f64": (None, [_f32p] * 5 + [_i64] * 3 + [_f64p]),
        "orc_matmul_f64": (None, [_f32p] * 3 + [_i64] * 3 + [_f64p]),
        "orc_relu_backward": (None, [_f32p] * 3 + [_i64]),
        "orc_sigmoid_backward": (None, [_f32p] * 3 + [_i64]),
        "orc_exp_backward": (None, [_f32p] * 3 + [_i64]),
        "orc_log_backward": (None, [_f32p] * 3 + [_i64]),
        "orc_tanh_backward": (None, [_f32p] * 3 + [_i64]),
        "orc_tan_backward": (None, [_f32p] * 3 + [_i64]),
        "orc_pow_backward": (None, [_f32p, _f32p, _f32, _f32p, _i64]),
        "orc_sqrt_backward": (None, [_f32p] * 3 + [_i64]),
        "orc_sin_backward": (None, [_f32p] * 3 + [_i64]),
        "orc_cos_backward": (None, [_f32p] * 3 + [_i64]),
        "orc_sub_backward": (None, [_f32p] * 3 + [_i64]),
        "orc_mul_backward": (None, [_f32p] * 5 + [_i64]),
        "orc_div_backward": (None, [_f32p] * 5 + [_i64]),
        "orc_sum_backward": (None, [_f32, _f32p, _i64]),
        "orc_mean_backward": (None, [_f32, _f32p, _i64]),
        "orc_mse_backward": (None, [_f32, _f32p, _f32p, _f32p, _f32p, _i64]),
        "orc_mse_loss": (_f32, [_f32p, _f32p, _i64]),
        "orc_mean_fwd": (_f32, [_f32p, _i64]),
        "orc_cross_entropy_backward": (None, [_f32, _f32p, _f32p, _f32p, _i64, _i64]),
        "orc_cross_entropy_loss": (_f32, [_f32p, _f32p, _i64, _i64]),
        "orc_softmax_backward": (None, [_f32p, _f32p, _f32p, _i64, _i64, _f32p]),
        "orc_unbroadcast_reference_accumulate": (None, [_f32p, _i64, _f32p]),
        "orc_sum_to_shape_f64": (ctypes.c_int, [_f32p, _i64p, ctypes.c_int, _f32p, _i64p,
                                                ctypes.c_int, _f64p]),
        "orc_powi": (_f32, [_f32, ctypes.c_int]),
        "orc_sgd_step": (None, [_f32p, _f32p, _f32p, _i64, _f32, _f32, _f32]),
        "orc_adam_step": (None, [_f32p, _f32p, _f32p, _f32p, _i64, _f32, _f32, _f32, _f32,
                                 _f32, ctypes.c_int]),
        "orc_argmax_rows": (None, [_f32p, _i64, _i64, _i32p, ctypes.c_int]),
        "orc_relu": (None, [_f32p, _f32p, _i64]),
        "orc_sigmoid": (None, [_f32p, _f32p, _i64]),
        "orc_gelu_backward_f64": (None, [_f32p] * 3 + [_i64]),
        "orc_gelu_f64": (None, [_f32p, _f32p, _i64]),
        "orc_layernorm_fwd_f64": (None, [_f32p] * 6 + [_i64, _i64, _f32]),
        "orc_layernorm_backward_f64": (None, [_f32p] * 6 + [_i64, _i64, _f32, _f64p]),
        "orc_softmax_rows_f64": (None, [_f32p, _f32p, _i64, _i64]),
        "orc_reduce_axis": (None, [_f32p, _i64, _i64, _i64, _i, _f32p]),
        "orc_elementwise": (None, [_i, _f32p, _f32p, _f32p, _i64]),
        "orc_reduction": (_i, [_i, _f32p, _i64p, _i, _i, _f32p]),
        "orc_broadcast_axis": (None, [_f32p, _i64, _i64, _i64, _i, _f32p]),
        "orc_softmax_axis_f64": (None, [_f32p, _i64, _i64, _i64, _f32p]),
        "orc_softmax_axis_backward_f64": (None, [_f32p, _f32p, _i64, _i64, _i64, _f32p]),
        "orc_softmax_backward_f64": (None, [_f32p] * 3 + [_i64, _i64]),
        "orc_adamw_step": (None, [_f32p] * 4 + [_i64] + [_f32] * 5 + [ctypes.c_int]),
        "orc_rmsprop_step": (None, [_f32p] * 4 + [_i64] + [_f32] * 5),
        "orc_adagrad_step": (None, [_f32p] * 3 + [_i64] + [_f32] * 3),
        "orc_nadam_step": (None, [_f32p] * 4 + [_i64] + [_f32] * 5 + [ctypes.c_int]),
        "orc_radam_step": (ctypes.c_int, [_f32p] * 4 + [_i64] + [_f32] * 5 + [ctypes.c_int]),
        "orc_adadelta_step": (None, [_f32p] * 4 + [_i64] + [_f32] * 3),
        "orc_adabound_step": (None, [_f32p] * 4 + [_i64] + [_f32] * 7 + [ctypes.c_int]),
        "orc_rprop_step": (None, [_f32p] * 4 + [_i64] + [_f32] * 4),
        "orc_lamb_step": (_f32, [_f32p] * 5 + [_i64] + [_f32] * 5 + [ctypes.c_int]),
        "orc_lookahead_sync": (None, [_f32p, _f32p, _i64, _f32]),
        "orc_dot_seq": (_f32, [_f32p, _f32p, _i64]),
        "orc_sched_step_lr": (_f32, [_f32p, _f32, ctypes.c_int, _f32]),
        "orc_sched_exponential": (_f32, [_f32p, _f32, _f32]),
        "orc_sched_cosine": (_f32, [_f32p, _f32, ctypes.c_int, _f32]),
        "orc_sched_plateau": (_f32, [_f32p, _f32, _f32, _f32, ctypes.c_int, _f32]),
        "orc_sched_warmup": (_f32, [_f32p, _f32, ctypes.c_int, _f32]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _p(a, ctype=_f32p):
    return None if a is None else a.ctypes.data_as(ctype)


def _f(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# --- reductions -------------------------------------------------------------

def sum_avx2_order(x) -> np.float32:
    x = _f(x)
    return np.float32(lib().orc_sum_avx2_order(_p(x), x.size))


def sum_seq(x) -> np.float32:
    x = _f(x)
    return np.float32(lib().orc_sum_seq(_p(x), x.size))


def sum_avx2_order_mt(x, threads: int) -> np.float32:
    """The full sum on `threads` host threads, each chunk in the 8-lane order
    (the all-cores CPU baseline of the reduction rows)."""
    x = _f(x)
    return np.float32(lib().orc_sum_avx2_order_mt(_p(x), x.size, int(threads)))


def transpose(x) -> np.ndarray:
    x = _f(x)
    r, c = x.shape
    y = np.empty((c, r), np.float32)
    lib().orc_transpose(_p(x), r, c, _p(y))
    return y


def accumulate(dst: np.ndarray, src) -> None:
    src = _f(src)
    lib().orc_accumulate(_p(dst), dst.size, _p(src), src.size)


# --- shape ops (no arithmetic: restated here in Python) ------------------------

def reshape_shape(total: int, new_shape) -> tuple:
    """ops::reshape's shape rules (ops/shape/reshape.rs:43-100): at most one
    -1, inferred as total / (product of the others); any other negative size,
    or a product that differs from `total`, raises ValueError."""
    infer, known = None, 1
    for i, d in enumerate(new_shape):
        d = int(d)
        if d == -1:
            if infer is not None:
                raise ValueError("Can only specify one unknown dimension with -1")
            infer = i
        elif d < 0:
            raise ValueError(f"Invalid dimension size: {d}")
        else:
            known *= d
    out = [int(d) for d in new_shape]
    if infer is not None:
        if known == 0:
            raise ValueError("Cannot infer dimension when other dimensions are zero")
        if total % known:
            raise ValueError(f"Cannot reshape array of size {total}")
        out[infer] = total // known
    elif known != total:
        raise ValueError(f"Cannot reshape array of size {total}")
    return tuple(out)


def flatten_shape(shape, start_dim: int, end_dim: int) -> tuple:
    """ops::flatten's output shape (ops/shape/flatten.rs:13-43): end_dim is
    clamped to the last dim, dims start_dim..=end_dim merge into one."""
    nd = len(shape)
    end = nd - 1 if end_dim >= nd else end_dim
    if start_dim > end:
        raise ValueError(f"flatten: start_dim ({start_dim}) cannot come after end_dim ({end})")
    flat = 1
    for i in range(start_dim, end + 1):
        flat *= int(shape[i])
    return tuple(int(s) for s in shape[:start_dim]) + (flat,) + tuple(int(s) for s in shape[end + 1:])


def reshape_backward(g, input_shape) -> np.ndarray:
    """reshape_backward / flatten_backward (backward.rs:315-330): the incoming
    grad, in row-major order, reshaped to the input's shape (a copy)."""
    g = _f(g)
    return g.reshape(reshape_shape(g.size, input_shape)).copy()


# --- matmul -----------------------------------------------------------------

def matmul_backward(dC, A, B, need_a=True, need_b=True, f64=False, rows_a=None, rows_b=None):
    """(dA, dB) = (dC @ B^T, A^T @ dC).  f64=False is the fp32 loop of
    backward.rs:123-146; f64=True accumulates in float64.  rows_a/rows_b
    restrict the computed rows (others stay NaN)."""
    dC, A, B = _f(dC), _f(A), _f(B)
    M, K = A.shape
    N = B.shape[1]
    assert B.shape[0] == K and dC.shape == (M, N)
    dA = np.full((M, K), np.nan, np.float32) if need_a else None
    dB = np.full((K, N), np.nan, np.float32) if need_b else None
    a0, a1 = rows_a if rows_a is not None else (0, M)
    b0, b1 = rows_b if rows_b is not None else (0, K)
    if f64:
        work = np.empty(max(K, N), np.float64)
        lib().orc_matmul_backward_f64_rows(_p(dC), _p(A), _p(B), _p(dA), _p(dB), M, K, N,
                                           a0, a1, b0, b1, _p(work, _f64p))
    else:
        lib().orc_matmul_backward_rows(_p(dC), _p(A), _p(B), _p(dA), _p(dB), M, K, N,
                                       a0, a1, b0, b1)
    return dA, dB


def matmul_f64(A, B) -> np.ndarray:
    A, B = _f(A), _f(B)
    M, K = A.shape
    N = B.shape[1]
    C = np.empty((M, N), np.float32)
    work = np.empty(N, np.float64)
    lib().orc_matmul_f64(_p(A), _p(B), _p(C), M, K, N, _p(work, _f64p))
    return C


# --- elementwise backward ---------------------------------------------------

def _unary(name, g, x):
    g, x = _f(g), _f(x)
    dx = np.empty_like(g)
    getattr(lib(), name)(_p(g), _p(x), _p(dx), g.size)
    return dx


def relu_backward(g, x):
    return _unary("orc_relu_backward", g, x)


def sigmoid_backward(g, s):
    return _unary("orc_sigmoid_backward", g, s)


def exp_backward(g, e):
    return _unary("orc_exp_backward", g, e)


def log_backward(g, x):
    return _unary("orc_log_backward", g, x)


def tanh_backward(g, y):
    return _unary("orc_tanh_backward", g, y)


def tan_backward(g, t):
    return _unary("orc_tan_backward", g, t)


def sqrt_backward(g, x):
    return _unary("orc_sqrt_backward", g, x)


def sin_backward(g, x):
    return _unary("orc_sin_backward", g, x)


def cos_backward(g, x):
    return _unary("orc_cos_backward", g, x)


def gelu_backward(g, x):
    return _unary("orc_gelu_backward_f64", g, x)


def pow_backward(g, x, expo):
    g, x = _f(g), _f(x)
    dx = np.empty_like(g)
    lib().orc_pow_backward(_p(g), _p(x), float(expo), _p(dx), g.size)
    return dx


def sub_backward(g):
    g = _f(g)
    dx, dy = np.empty_like(g), np.empty_like(g)
    lib().orc_sub_backward(_p(g), _p(dx), _p(dy), g.size)
    return dx, dy


def mul_backward(g, x, y):
    g, x, y = _f(g), _f(x), _f(y)
    dx, dy = np.empty_like(g), np.empty_like(g)
    lib().orc_mul_backward(_p(g), _p(x), _p(y), _p(dx), _p(dy), g.size)
    return dx, dy


def div_backward(g, x, y):
    g, x, y = _f(g), _f(x), _f(y)
    dx, dy = np.empty_like(g), np.empty_like(g)
    lib().orc_div_backward(_p(g), _p(x), _p(y), _p(dx), _p(dy), g.size)
    return dx, dy


def sum_backward(g0, shape):
    dx = np.empty(shape, np.float32)
    lib().orc_sum_backward(float(g0), _p(dx), dx.size)
    return dx


def mean_backward(g0, shape):
    dx = np.empty(shape, np.float32)
    lib().orc_mean_backward(float(g0), _p(dx), dx.size)
    return dx


def mse_backward(g0, p, t):
    p, t = _f(p), _f(t)
    dp, dt = np.empty_like(p), np.empty_like(p)
    lib().orc_mse_backward(float(g0), _p(p), _p(t), _p(dp), _p(dt), p.size)
    return dp, dt


def mse_loss(p, t) -> np.float32:
    p, t = _f(p), _f(t)
    return np.float32(lib().orc_mse_loss(_p(p), _p(t), p.size))


def mean_fwd(x) -> np.float32:
    x = _f(x)
    return np.float32(lib().orc_mean_fwd(_p(x), x.size))


def cross_entropy_backward(g0, logits, onehot):
    x, t = _f(logits), _f(onehot)
    B, C = x.shape
    dx = np.empty_like(x)
    lib().orc_cross_entropy_backward(float(g0), _p(x), _p(t), _p(dx), B, C)
    return dx


def cross_entropy_loss(logits, onehot) -> np.float32:
    x, t = _f(logits), _f(onehot)
    B, C = x.shape
    return np.float32(lib().orc_cross_entropy_loss(_p(x), _p(t), B, C))


def softmax_backward(y, g, f64=False):
    y, g = _f(y), _f(g)
    rows, cols = y.shape
    dx = np.empty_like(y)
    if f64:
        lib().orc_softmax_backward_f64(_p(y), _p(g), _p(dx), rows, cols)
    else:
        work = np.empty(cols, np.float32)
        lib().orc_softmax_backward(_p(y), _p(g), _p(dx), rows, cols, _p(work))
    return dx


def softmax_rows(x):
    x = _f(x)
    rows, cols = x.shape
    y = np.empty_like(x)
    lib().orc_softmax_rows_f64(_p(x), _p(y), rows, cols)
    return y


# --- DispatchTable forward kernels ----------------------------------------------

def elementwise(kind: int, a, b=None):
    """elementwise_scalar(a, b, kind) (backend/cpu/scalar.rs:11-150)."""
    a = _f(a)
    bb = None if b is None else _f(b)
    out = np.empty_like(a)
    lib().orc_elementwise(kind, _p(a), _p(bb), _p(out), a.size)
    return out


def reduction(kind: int, x, axis=None):
    """reduce_scalar(a, axis, kind) (backend/cpu/scalar.rs:495-788)."""
    x = _f(x)
    shape = np.array(x.shape, np.int64)
    if axis is None:
        out = np.empty(1, np.float32)
    else:
        out = np.empty(_axis_out_shape(x.shape, axis), np.float32)
    rc = lib().orc_reduction(kind, _p(x), _p(shape, _i64p), x.ndim,
                             -1 if axis is None else int(axis), _p(out))
    if rc != 0:
        raise ValueError("bad reduction arguments")
    return out


# --- axis reductions and axis softmax -------------------------------------------

def axis_view(shape, axis):
    """(outer, n, inner) of `shape` around `axis`."""
    outer = int(np.prod(shape[:axis], dtype=np.int64))
    inner = int(np.prod(shape[axis + 1:], dtype=np.int64))
    return outer, int(shape[axis]), inner


def _axis_out_shape(shape, axis):
    s = tuple(d for k, d in enumerate(shape) if k != axis)
    return s if s else (1,)


def reduce_axis(x, axis, mean=False):
    """ops::sum / ops::mean with Some(axis) (scalar.rs:584-788): the axis removed."""
    x = _f(x)
    o, n, i = axis_view(x.shape, axis)
    out = np.empty(_axis_out_shape(x.shape, axis), np.float32)
    lib().orc_reduce_axis(_p(x), o, n, i, int(mean), _p(out))
    return out


def broadcast_axis(g, shape, axis, mean=False):
    """Backward of reduce_axis: g broadcast back along the axis (divided by n for the mean)."""
    g = _f(g)
    o, n, i = axis_view(shape, axis)
    dx = np.empty(shape, np.float32)
    lib().orc_broadcast_axis(_p(g), o, n, i, int(mean), _p(dx))
    return dx


def softmax_axis(x, axis):
    x = _f(x)
    o, n, i = axis_view(x.shape, axis)
    y = np.empty_like(x)
    lib().orc_softmax_axis_f64(_p(x), o, n, i, _p(y))
    return y


def softmax_axis_backward(y, g, axis):
    y, g = _f(y), _f(g)
    o, n, i = axis_view(y.shape, axis)
    dx = np.empty_like(y)
    lib().orc_softmax_axis_backward_f64(_p(y), _p(g), o, n, i, _p(dx))
    return dx


# --- unbroadcast --------------------------------------------------------------

def unbroadcast_reference_accumulate(g, out_grad: np.ndarray) -> None:
    """REFERENCE mode (backward.rs:12-39 + tensor.rs:120-132): sum into element 0."""
    g = _f(g)
    lib().orc_unbroadcast_reference_accumulate(_p(g), g.size, _p(out_grad))


def sum_to_shape(g, shape):
    g = _f(g)
    gshape = np.array(g.shape, np.int64)
    oshape = np.array(shape, np.int64)
    out = np.empty(shape, np.float32)
    work = np.empty(max(out.size, 1), np.float64)
    rc = lib().orc_sum_to_shape_f64(_p(g), _p(gshape, _i64p), g.ndim, _p(out),
                                    _p(oshape, _i64p), len(shape), _p(work, _f64p))
    if rc != 0:
        raise ValueError(f"cannot sum {g.shape} to {tuple(shape)}")
    return out


# --- optimizers -----------------------------------------------------------------

def powi(a: float, t: int) -> np.float32:
    return np.float32(lib().orc_powi(float(a), int(t)))


def sgd_step(p: np.ndarray, g, v: np.ndarray | None, lr, mu=0.0, wd=0.0) -> None:
    g = _f(g)
    lib().orc_sgd_step(_p(p), _p(g), _p(v), p.size, lr, mu, wd)


def adam_step(p: np.ndarray, g, m: np.ndarray, v: np.ndarray, t: int, lr=1e-3, b1=0.9,
              b2=0.999, eps=1e-8, wd=0.0) -> None:
    g = _f(g)
    lib().orc_adam_step(_p(p), _p(g), _p(m), _p(v), p.size, lr, b1, b2, eps, wd, int(t))


def _st(x):
    return None if x is None else _p(x)


def adamw_step(p, g, m, v, t, lr, b1=0.9, b2=0.999, eps=1e-8, wd=0.01):
    lib().orc_adamw_step(_p(p), _p(_f(g)), _p(m), _p(v), p.size, lr, b1, b2, eps, wd, int(t))


def rmsprop_step(p, g, v, buf, lr, alpha=0.99, eps=1e-8, wd=0.0, momentum=0.0):
    lib().orc_rmsprop_step(_p(p), _p(_f(g)), _p(v), _p(buf), p.size, lr, alpha, eps, wd, momentum)


def adagrad_step(p, g, acc, lr, eps=1e-10, wd=0.0):
    lib().orc_adagrad_step(_p(p), _p(_f(g)), _p(acc), p.size, lr, eps, wd)


def nadam_step(p, g, m, v, t, lr, b1=0.9, b2=0.999, eps=1e-8, wd=0.0):
    lib().orc_nadam_step(_p(p), _p(_f(g)), _p(m), _p(v), p.size, lr, b1, b2, eps, wd, int(t))


def radam_step(p, g, m, v, t, lr, b1=0.9, b2=0.999, eps=1e-8, wd=0.0) -> bool:
    return bool(lib().orc_radam_step(_p(p), _p(_f(g)), _p(m), _p(v), p.size, lr, b1, b2, eps, wd,
                                     int(t)))


def adadelta_step(p, g, eg, ed, rho=0.95, eps=1e-6, wd=0.0):
    lib().orc_adadelta_step(_p(p), _p(_f(g)), _p(eg), _p(ed), p.size, rho, eps, wd)


def adabound_step(p, g, m, v, t, lr, final_lr=0.1, b1=0.9, b2=0.999, eps=1e-8, wd=0.0,
                  gamma=0.001):
    lib().orc_adabound_step(_p(p), _p(_f(g)), _p(m), _p(v), p.size, lr, final_lr, b1, b2, eps,
                            wd, gamma, int(t))


def rprop_step(p, g, step, prev, eta_plus=1.2, eta_minus=0.5, lr_min=1e-6, lr_max=50.0):
    lib().orc_rprop_step(_p(p), _p(_f(g)), _p(step), _p(prev), p.size, eta_plus, eta_minus,
                         lr_min, lr_max)


def lamb_step(p, g, m, v, t, lr, b1=0.9, b2=0.999, eps=1e-6, wd=0.01) -> np.float32:
    u = np.empty_like(p)
    return np.float32(lib().orc_lamb_step(_p(p), _p(_f(g)), _p(m), _p(v), _p(u), p.size, lr, b1,
                                          b2, eps, wd, int(t)))


def lookahead_sync(fast, slow, alpha):
    lib().orc_lookahead_sync(_p(fast), _p(slow), fast.size, alpha)


def dot_seq(a, b) -> np.float32:
    a, b = _f(a), _f(b)
    return np.float32(lib().orc_dot_seq(_p(a), _p(b), a.size))


class Scheduler:
    """optim/schedulers.rs restated over a plain learning-rate value."""

    def __init__(self, kind: str, *args):
        self.kind, self.args = kind, args
        self.st = np.zeros(6, np.float32)

    def step(self, lr, metric=None) -> np.float32:
        L, st, a = lib(), _p(self.st), self.args
        if self.kind == "step":
            return np.float32(L.orc_sched_step_lr(st, lr, int(a[0]), a[1]))
        if self.kind == "exponential":
            return np.float32(L.orc_sched_exponential(st, lr, a[0]))
        if self.kind == "cosine":
            return np.float32(L.orc_sched_cosine(st, lr, int(a[0]), a[1]))
        if self.kind == "plateau":
            return np.float32(L.orc_sched_plateau(st, lr, metric, a[0], int(a[1]), a[2]))
        if self.kind == "warmup":
            return np.float32(L.orc_sched_warmup(st, lr, int(a[0]), a[1]))
        raise ValueError(self.kind)


class LBFGS:
    """L-BFGS over flattened parameters, optim/lbfgs.rs:38-212: two-loop
    recursion with f32 scalars and sequential f32 dot products (orc_dot_seq)."""

    def __init__(self, lr=1.0, history_size=10):
        self.lr, self.h = np.float32(lr), history_size
        self.s, self.y = [], []
        self.prev_p = self.prev_g = None

    def _dir(self, g):
        f = np.float32
        if not self.s:
            return -g
        m = len(self.s)
        q = g.copy()
        alpha, rho = [f(0)] * m, [f(0)] * m
        for i in reversed(range(m)):
            rho[i] = f(1.0) / max(dot_seq(self.y[i], self.s[i]), f(1e-10))
            alpha[i] = rho[i] * dot_seq(self.s[i], q)
            q = (q - alpha[i] * self.y[i]).astype(np.float32)
        gamma = dot_seq(self.s[-1], self.y[-1]) / max(dot_seq(self.y[-1], self.y[-1]), f(1e-10))
        r = (gamma * q).astype(np.float32)
        for i in range(m):
            beta = rho[i] * dot_seq(self.y[i], r)
            r = (r + self.s[i] * f(alpha[i] - beta)).astype(np.float32)
        return -r

    def step(self, params: list, grads: list) -> None:
        cur_p = np.concatenate([x.ravel() for x in params]).astype(np.float32)
        cur_g = np.concatenate([x.ravel() for x in grads]).astype(np.float32)
        if self.prev_p is not None:
            s = (cur_p - self.prev_p).astype(np.float32)
            y = (cur_g - self.prev_g).astype(np.float32)
            if dot_seq(s, y) > np.float32(1e-10):
                self.s.append(s)
                self.y.append(y)
                if len(self.s) > self.h:
                    self.s.pop(0)
                    self.y.pop(0)
        d = self._dir(cur_g)
        off = 0
        for x in params:
            n = x.size
            x.ravel()[:] = (x.ravel() + self.lr * d[off:off + n]).astype(np.float32)
            off += n
        self.prev_p, self.prev_g = cur_p, cur_g


# --- integer paths ----------------------------------------------------------------

def argmax_rows(x, tie_last=False) -> np.ndarray:
    x = _f(x)
    rows, cols = x.shape
    idx = np.empty(rows, np.int32)
    lib().orc_argmax_rows(_p(x), rows, cols, _p(idx, _i32p), int(tie_last))
    return idx


# --- forward helpers -----------------------------------------------------------------

def relu(x):
    x = _f(x)
    y = np.empty_like(x)
    lib().orc_relu(_p(x), _p(y), x.size)
    return y


def sigmoid(x):
    x = _f(x)
    y = np.empty_like(x)
    lib().orc_sigmoid(_p(x), _p(y), x.size)
    return y


def gelu(x):
    x = _f(x)
    y = np.empty_like(x)
    lib().orc_gelu_f64(_p(x), _p(y), x.size)
    return y


def layernorm_fwd(x, gamma, beta, eps=1e-5):
    x, gamma, beta = _f(x), _f(gamma), _f(beta)
    rows, cols = x.shape
    y = np.empty_like(x)
    mean = np.empty(rows, np.float32)
    rstd = np.empty(rows, np.float32)
    lib().orc_layernorm_fwd_f64(_p(x), _p(gamma), _p(beta), _p(y), _p(mean), _p(rstd),
                                rows, cols, eps)
    return y, mean, rstd


def layernorm_backward(g, x, gamma, eps=1e-5):
    g, x, gamma = _f(g), _f(x), _f(gamma)
    rows, cols = x.shape
    dx = np.empty_like(x)
    dgamma = np.empty(cols, np.float32)
    dbeta = np.empty(cols, np.float32)
    work = np.empty(2 * cols, np.float64)
    lib().orc_layernorm_backward_f64(_p(g), _p(x), _p(gamma), _p(dx), _p(dgamma), _p(dbeta),
                                     rows, cols, eps, _p(work, _f64p))
    return dx, dgamma, dbeta
