"""Optimizers and LR schedulers over device parameters (mirrors
numrs-core/src/autograd/optim).

Every optimizer keeps its state (velocities, moments, step sizes, L-BFGS
history) on the device and updates all of its parameters with one fused
multi-tensor launch per step; the schedulers are host state machines that
read and set the optimizer's learning rate.
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

    def state_info(self) -> tuple[int, int, int]:
        """(parameters, state slots per parameter, step counter) for checkpoints."""
        n, k, t = ctypes.c_int(), ctypes.c_int(), ctypes.c_int64()
        self.ctx._check(L.load().numrs_hip_optim_state_info(self._h, ctypes.byref(n),
                                                            ctypes.byref(k), ctypes.byref(t)))
        return n.value, k.value, t.value

    def get_state(self, param: int, slot: int):
        """One state slot of one parameter as a float32 array of the parameter's shape."""
        import numpy as np

        shape = self._params[param].shape()
        out = np.empty(shape, np.float32)
        self.ctx._check(L.load().numrs_hip_optim_state_get(self._h, param, slot,
                                                           out.ctypes.data, out.size))
        return out

    def set_state(self, param: int, slot: int, values) -> None:
        import numpy as np

        arr = np.ascontiguousarray(values, np.float32).ravel()
        self.ctx._check(L.load().numrs_hip_optim_state_set(self._h, param, slot,
                                                           arr.ctypes.data, arr.size))

    def set_step(self, step: int) -> None:
        self.ctx._check(L.load().numrs_hip_optim_set_step(self._h, int(step)))

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
    """SGD::new(params, lr, momentum, weight_decay) (optim/sgd.rs:47-69)."""

    def __init__(self, params, lr: float, momentum: float = 0.0, weight_decay: float = 0.0):
        params = list(params)
        ctx = params[0].ctx
        arr, n = _handles(params)
        h = ctypes.c_void_p()
        ctx._check(L.load().numrs_hip_optim_sgd(ctx.handle, arr, n, lr, momentum, weight_decay,
                                                ctypes.byref(h)))
        super().__init__(h.value, ctx, params)
        # OptimizerKind::SGD (llo/model.rs:31) and the names of the state slots
        self._ckpt = ("SGD", {"momentum": momentum}, ("velocity",))

    @classmethod
    def simple(cls, params, lr: float) -> "SGD":
        """SGD::simple (sgd.rs:71-73)."""
        return cls(params, lr, 0.0, 0.0)


class Adam(Optimizer):
    """Adam::new(params, lr, beta1, beta2, eps, weight_decay) (optim/adam.rs:64-99)."""

    def __init__(self, params, lr: float, beta1: float = 0.9, beta2: float = 0.999,
                 eps: float = 1e-8, weight_decay: float = 0.0):
        params = list(params)
        ctx = params[0].ctx
        arr, n = _handles(params)
        h = ctypes.c_void_p()
        ctx._check(L.load().numrs_hip_optim_adam(ctx.handle, arr, n, lr, beta1, beta2, eps,
                                                 weight_decay, ctypes.byref(h)))
        super().__init__(h.value, ctx, params)
        self._ckpt = ("Adam", {"beta1": beta1, "beta2": beta2, "epsilon": eps}, ("m", "v"))

    @classmethod
    def default(cls, params, lr: float) -> "Adam":
        """Adam::default (adam.rs:102-104)."""
        return cls(params, lr)


def _kind_optim(kind: int, params, hyper) -> tuple:
    params = list(params)
    ctx = params[0].ctx
    arr, n = _handles(params)
    hv = (ctypes.c_float * len(hyper))(*[float(x) for x in hyper])
    h = ctypes.c_void_p()
    ctx._check(L.load().numrs_hip_optim_create(ctx.handle, kind, arr, n, hv, len(hyper),
                                               ctypes.byref(h)))
    return h.value, ctx, params


class AdamW(Optimizer):
    """AdamW::new(params, lr, beta1, beta2, eps, weight_decay) (optim/adamw.rs:50-83)."""

    def __init__(self, params, lr: float, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01):
        super().__init__(*_kind_optim(L.OPT_ADAMW, params, (lr, beta1, beta2, eps, weight_decay)))

    @classmethod
    def default(cls, params, lr: float) -> "AdamW":  # adamw.rs:86-88
        return cls(params, lr)


class RMSprop(Optimizer):
    """RMSprop::new(params, lr, alpha, eps, weight_decay, momentum) (optim/rmsprop.rs:47-81)."""

    def __init__(self, params, lr: float, alpha=0.99, eps=1e-8, weight_decay=0.0, momentum=0.0):
        super().__init__(*_kind_optim(L.OPT_RMSPROP, params,
                                      (lr, alpha, eps, weight_decay, momentum)))
        self._ckpt = ("RMSprop", {"decay": alpha, "epsilon": eps},
                      ("square_avg", "momentum_buffer"))

    @classmethod
    def default(cls, params, lr: float) -> "RMSprop":  # rmsprop.rs:84-86
        return cls(params, lr)


class AdaGrad(Optimizer):
    """AdaGrad::new(params, lr, eps, weight_decay) (optim/adagrad.rs:43-63)."""

    def __init__(self, params, lr: float, eps=1e-10, weight_decay=0.0):
        super().__init__(*_kind_optim(L.OPT_ADAGRAD, params, (lr, eps, weight_decay)))
        self._ckpt = ("AdaGrad", {"epsilon": eps}, ("sum_sq",))

    @classmethod
    def default(cls, params, lr: float) -> "AdaGrad":  # adagrad.rs:66-68
        return cls(params, lr)


class NAdam(Optimizer):
    """NAdam::new(params, lr, beta1, beta2, eps, weight_decay) (optim/nadam.rs:57-90)."""

    def __init__(self, params, lr: float, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0):
        super().__init__(*_kind_optim(L.OPT_NADAM, params, (lr, beta1, beta2, eps, weight_decay)))

    @classmethod
    def default(cls, params, lr: float) -> "NAdam":  # nadam.rs:93-95
        return cls(params, lr)


class RAdam(Optimizer):
    """RAdam::new(params, lr, beta1, beta2, eps, weight_decay) (optim/radam.rs:53-86)."""

    def __init__(self, params, lr: float, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0):
        super().__init__(*_kind_optim(L.OPT_RADAM, params, (lr, beta1, beta2, eps, weight_decay)))

    @classmethod
    def default(cls, params, lr: float) -> "RAdam":  # radam.rs:89-91
        return cls(params, lr)


class AdaDelta(Optimizer):
    """AdaDelta::new(params, rho, eps, weight_decay) (optim/adadelta.rs:53-81); no
    learning rate: learning_rate() reads 1.0 and set_learning_rate is ignored."""

    def __init__(self, params, rho=0.95, eps=1e-6, weight_decay=0.0):
        super().__init__(*_kind_optim(L.OPT_ADADELTA, params, (rho, eps, weight_decay)))

    @classmethod
    def default(cls, params) -> "AdaDelta":  # adadelta.rs:84-86
        return cls(params)


class AdaBound(Optimizer):
    """AdaBound::new(params, lr, final_lr, beta1, beta2, eps, weight_decay, gamma)
    (optim/adabound.rs:70-107)."""

    def __init__(self, params, lr: float, final_lr=0.1, beta1=0.9, beta2=0.999, eps=1e-8,
                 weight_decay=0.0, gamma=0.001):
        super().__init__(*_kind_optim(L.OPT_ADABOUND, params,
                                      (lr, final_lr, beta1, beta2, eps, weight_decay, gamma)))

    @classmethod
    def default(cls, params, lr: float) -> "AdaBound":  # adabound.rs:110-112
        return cls(params, lr)


class Rprop(Optimizer):
    """Rprop::new(params, lr_init, eta_plus, eta_minus, lr_min, lr_max) (optim/rprop.rs:63-94);
    learning_rate() is the mean step size, set_learning_rate resets every step size."""

    def __init__(self, params, lr_init=0.01, eta_plus=1.2, eta_minus=0.5, lr_min=1e-6,
                 lr_max=50.0):
        super().__init__(*_kind_optim(L.OPT_RPROP, params,
                                      (lr_init, eta_plus, eta_minus, lr_min, lr_max)))

    @classmethod
    def default(cls, params) -> "Rprop":  # rprop.rs:97-99
        return cls(params)


class LAMB(Optimizer):
    """LAMB::new(params, lr, beta1, beta2, eps, weight_decay) (optim/lamb.rs:63-96)."""

    def __init__(self, params, lr: float, beta1=0.9, beta2=0.999, eps=1e-6, weight_decay=0.01):
        super().__init__(*_kind_optim(L.OPT_LAMB, params, (lr, beta1, beta2, eps, weight_decay)))

    @classmethod
    def default(cls, params, lr: float) -> "LAMB":  # lamb.rs:99-101
        return cls(params, lr)


class Lookahead(Optimizer):
    """Lookahead::new(inner, params, k, alpha) (optim/lookahead.rs:59-84).  The inner
    optimizer's handle is taken over: it is freed with the Lookahead."""

    def __init__(self, inner: Optimizer, params, k: int = 5, alpha: float = 0.5):
        params = list(params)
        ctx = inner.ctx
        arr, n = _handles(params)
        h = ctypes.c_void_p()
        ctx._check(L.load().numrs_hip_optim_lookahead(inner._h, arr, n, k, alpha,
                                                      ctypes.byref(h)))
        inner._h = None  # owned by the Lookahead now
        self.inner = inner
        super().__init__(h.value, ctx, params)


class LBFGS(Optimizer):
    """LBFGS::new(params, lr, history_size, max_iter) (optim/lbfgs.rs:60-76)."""

    def __init__(self, params, lr: float = 1.0, history_size: int = 10, max_iter: int = 20):
        params = list(params)
        ctx = params[0].ctx
        arr, n = _handles(params)
        h = ctypes.c_void_p()
        ctx._check(L.load().numrs_hip_optim_lbfgs(ctx.handle, arr, n, lr, history_size, max_iter,
                                                  ctypes.byref(h)))
        super().__init__(h.value, ctx, params)

    @classmethod
    def default(cls, params) -> "LBFGS":  # lbfgs.rs:79-81
        return cls(params)


# ---------------------------------------------------------------------------
# LR schedulers (optim/schedulers.rs)
# ---------------------------------------------------------------------------

class Scheduler:
    """trait Scheduler: step(optimizer), get_lr()."""

    def __init__(self, kind: int, hyper):
        hv = (ctypes.c_float * len(hyper))(*[float(x) for x in hyper])
        h = ctypes.c_void_p()
        rc = L.load().numrs_hip_scheduler_create(kind, hv, len(hyper), ctypes.byref(h))
        if rc != 0:
            raise ValueError(f"bad scheduler arguments {hyper}")
        self._h = h.value

    def step(self, optimizer: Optimizer) -> None:
        rc = L.load().numrs_hip_scheduler_step(self._h, optimizer._h)
        if rc != 0:
            raise RuntimeError("scheduler step refused (ReduceLROnPlateau needs step_with_metric)")

    def get_lr(self) -> float:
        return float(L.load().numrs_hip_scheduler_get_lr(self._h))

    def __del__(self):
        try:
            if self._h:
                L.load().numrs_hip_scheduler_free(self._h)
                self._h = None
        except Exception:
            pass


class StepLR(Scheduler):
    def __init__(self, step_size: int, gamma: float):  # schedulers.rs:33-40
        super().__init__(L.SCHED_STEP, (step_size, gamma))


class ExponentialLR(Scheduler):
    def __init__(self, gamma: float):  # schedulers.rs:79-85
        super().__init__(L.SCHED_EXPONENTIAL, (gamma,))


class CosineAnnealingLR(Scheduler):
    def __init__(self, t_max: int, eta_min: float):  # schedulers.rs:126-133
        super().__init__(L.SCHED_COSINE, (t_max, eta_min))


class ReduceLROnPlateau(Scheduler):
    def __init__(self, factor: float, patience: int, min_lr: float):  # schedulers.rs:189-198
        super().__init__(L.SCHED_PLATEAU, (factor, patience, min_lr))

    def step_with_metric(self, metric: float, optimizer: Optimizer) -> None:
        if L.load().numrs_hip_scheduler_step_metric(self._h, metric, optimizer._h) != 0:
            raise RuntimeError("scheduler step failed")


class LinearWarmup(Scheduler):
    def __init__(self, warmup_steps: int, start_lr: float):  # schedulers.rs:262-269
        super().__init__(L.SCHED_WARMUP, (warmup_steps, start_lr))
