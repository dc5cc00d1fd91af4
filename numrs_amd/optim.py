"""Optimizers over device parameters (mirrors numrs-core/src/autograd/optim).

Both keep their state (SGD velocities, Adam moments and step counter) on the
device and update every parameter with one fused kernel per tensor
(numrs_hip_sgd_step / numrs_hip_adam_step).
"""
from __future__ import annotations

import ctypes

from . import _lib as L
from .autograd import Tensor


class Optimizer:
    """trait Optimizer (optim/base.rs:8-23)."""

    def __init__(self, handle: int, ctx, params):
        self._h = handle
        self.ctx = ctx
        self._params = list(params)  # keep the handles alive

    def step(self) -> None:
        self.ctx._check(L.load().numrs_hip_optim_step(self._h))

    def zero_grad(self) -> None:
        self.ctx._check(L.load().numrs_hip_optim_zero_grad(self._h))

    def learning_rate(self) -> float:
        return float(L.load().numrs_hip_optim_lr(self._h))

    def set_learning_rate(self, lr: float) -> None:
        self.ctx._check(L.load().numrs_hip_optim_set_lr(self._h, lr))

    def num_params(self) -> int:
        return len(self._params)

    def __del__(self):
        try:
            if self._h:
                L.load().numrs_hip_optim_free(self._h)
                self._h = None
        except Exception:
            pass


def _handles(params: list[Tensor]):
    arr = (ctypes.c_void_p * max(len(params), 1))(*[p._h for p in params])
    return arr, len(params)


class SGD(Optimizer):
    """SGD::new(params, lr, momentum, weight_decay) (optim/sgd.rs:90-112)."""

    def __init__(self, params, lr: float, momentum: float = 0.0, weight_decay: float = 0.0):
        params = list(params)
        ctx = params[0].ctx
        arr, n = _handles(params)
        h = ctypes.c_void_p()
        ctx._check(L.load().numrs_hip_optim_sgd(ctx.handle, arr, n, lr, momentum, weight_decay,
                                                ctypes.byref(h)))
        super().__init__(h.value, ctx, params)

    @classmethod
    def simple(cls, params, lr: float) -> "SGD":
        """SGD::simple (sgd.rs:114-116)."""
        return cls(params, lr, 0.0, 0.0)


class Adam(Optimizer):
    """Adam::new(params, lr, beta1, beta2, eps, weight_decay) (optim/adam.rs:250-285)."""

    def __init__(self, params, lr: float, beta1: float = 0.9, beta2: float = 0.999,
                 eps: float = 1e-8, weight_decay: float = 0.0):
        params = list(params)
        ctx = params[0].ctx
        arr, n = _handles(params)
        h = ctypes.c_void_p()
        ctx._check(L.load().numrs_hip_optim_adam(ctx.handle, arr, n, lr, beta1, beta2, eps,
                                                 weight_decay, ctypes.byref(h)))
        super().__init__(h.value, ctx, params)

    @classmethod
    def default(cls, params, lr: float) -> "Adam":
        """Adam::default (adam.rs:288-290)."""
        return cls(params, lr)
