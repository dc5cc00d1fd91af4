"""numrs's JSON training checkpoint for device-resident parameters and
optimizer state.

The file is what numrs's `save_checkpoint` writes (ops/model.rs:544-588):
serde_json of `{ "model": OnnxModel, "training_state": TrainingState }`
(llo/model.rs).  Parameters are the model graph's initializers
(`OnnxTensor { name, dtype: 1 (FLOAT), shape, data: little-endian f32 bytes }`,
ops/model.rs:150-176); `TrainingState` carries epoch, iteration, loss, the
optimizer's `OptimizerKind` (externally tagged, as serde writes an enum),
the parameters' gradients and `optimizer_state` -- which numrs defines but
never fills; here it holds each parameter's state slots under
"<name>.<slot>" and the step counter under "step".

`OptimizerKind` names four families (SGD, Adam, RMSprop, AdaGrad); the
optimizers outside them cannot be written in this format and are refused.
Weight decay is not part of `OptimizerKind`: pass the same constructor
arguments when re-creating the optimizer before `restore`.
"""
from __future__ import annotations

import json
import math
from dataclasses import dataclass, field

import numpy as np

from .autograd import Tensor
from .device import DeviceArray

PRODUCER_VERSION = "0.1.23"  # numrs-core/Cargo.toml: the version serde writes via env!()
ONNX_FLOAT, ONNX_DOUBLE = 1, 11


def _f(v) -> float | None:
    """An f32 as serde_json writes it: finite values round-trip, NaN/inf become null."""
    v = float(np.float32(v))
    return v if math.isfinite(v) else None


def _floats(a) -> list:
    return [_f(v) for v in np.asarray(a, np.float32).ravel()]


def _tensor_json(name: str, values: np.ndarray) -> dict:
    arr = np.ascontiguousarray(values, "<f4")
    return {"name": name, "dtype": ONNX_FLOAT, "shape": [int(d) for d in arr.shape],
            "data": list(arr.tobytes())}


def _model_json(name: str, params: dict) -> dict:
    """OnnxModel::new(name) (llo/model.rs:158-173) with the parameters as initializers."""
    meta = {"name": name, "version": 1, "author": "NumRs",
            "description": "Model created with NumRs", "domain": "ai.numrs", "opset_version": 18,
            "producer_name": "NumRs", "producer_version": PRODUCER_VERSION, "metadata": {}}
    inits = [_tensor_json(k, v.values()) for k, v in params.items()]
    return {"metadata": meta,
            "graph": {"name": name, "nodes": [], "inputs": [], "outputs": [],
                      "initializers": inits}}


def _name_of(params: dict, t: Tensor) -> str:
    ptr = t.device_ptrs()[0]
    for k, v in params.items():
        if v.device_ptrs()[0] == ptr:
            return k
    raise ValueError("an optimizer parameter is missing from the checkpoint's parameter dict")


def save_checkpoint(path: str, params: dict, optimizer=None, *, epoch: int = 0,
                    iteration: int = 0, loss: float = 0.0, name: str = "numrs_model",
                    gradients: bool = True) -> None:
    """save_checkpoint(model, training_state, path) (ops/model.rs:550-569) for
    the named device tensors in `params` and the optimizer's state."""
    state: dict = {"epoch": int(epoch), "iteration": int(iteration), "loss": _f(loss)}
    opt_state: dict = {}
    if optimizer is None:
        # TrainingState::new_sgd(0.0) shape: a kind is required by the format.
        state["optimizer"] = {"SGD": {"learning_rate": 0.0, "momentum": 0.0}}
    else:
        ck = getattr(optimizer, "_ckpt", None)
        if ck is None:
            raise ValueError(f"{type(optimizer).__name__} has no OptimizerKind variant in numrs's "
                             "checkpoint format (SGD, Adam, RMSprop, AdaGrad)")
        variant, fields, slot_names = ck
        state["optimizer"] = {variant: {"learning_rate": _f(optimizer.learning_rate()),
                                        **{k: _f(v) for k, v in fields.items()}}}
        n, slots, step = optimizer.state_info()
        for i in range(n):
            pname = _name_of(params, optimizer._params[i])
            for s in range(slots):
                try:
                    vals = optimizer.get_state(i, s)
                except Exception:
                    continue  # this parameter has no such slot (e.g. RMSprop without momentum)
                opt_state[f"{pname}.{slot_names[s]}"] = _floats(vals)
        opt_state["step"] = [float(step)]
    grads: dict = {}
    if gradients:
        for k, t in params.items():
            g = t.gradient()
            if g is not None:
                grads[k] = _floats(g)
    state["gradients"] = grads
    state["optimizer_state"] = opt_state
    doc = {"model": _model_json(name, params), "training_state": state}
    with open(path, "w") as f:
        json.dump(doc, f, indent=2)


@dataclass
class Checkpoint:
    """load_checkpoint(path) -> (OnnxModel, TrainingState) (ops/model.rs:577-588)."""
    name: str
    initializers: dict
    epoch: int
    iteration: int
    loss: float
    optimizer: dict
    gradients: dict = field(default_factory=dict)
    optimizer_state: dict = field(default_factory=dict)


def _array(t: dict) -> np.ndarray:
    raw = bytes(t["data"])
    if t["dtype"] == ONNX_FLOAT:
        a = np.frombuffer(raw, "<f4")
    elif t["dtype"] == ONNX_DOUBLE:
        a = np.frombuffer(raw, "<f8").astype(np.float32)
    else:
        raise ValueError(f"initializer {t['name']!r}: ONNX dtype {t['dtype']} is not a float type")
    shape = tuple(int(d) for d in t["shape"])
    if a.size != int(np.prod(shape, dtype=np.int64)):
        raise ValueError(f"initializer {t['name']!r}: {a.size} values for shape {shape}")
    return a.reshape(shape).copy()


def _vals(v) -> np.ndarray:
    return np.array([np.nan if x is None else x for x in v], np.float32)


def load_checkpoint(path: str) -> Checkpoint:
    with open(path) as f:
        doc = json.load(f)
    model, ts = doc["model"], doc["training_state"]
    inits = {t["name"]: _array(t) for t in model["graph"]["initializers"]}
    return Checkpoint(name=model["metadata"]["name"], initializers=inits,
                      epoch=int(ts["epoch"]), iteration=int(ts["iteration"]),
                      loss=float("nan") if ts["loss"] is None else float(ts["loss"]),
                      optimizer=ts["optimizer"],
                      gradients={k: _vals(v) for k, v in ts.get("gradients", {}).items()},
                      optimizer_state={k: _vals(v)
                                       for k, v in ts.get("optimizer_state", {}).items()})


def restore(ckpt: Checkpoint, params: dict, optimizer=None) -> None:
    """Uploads the checkpoint's parameter values (and, with an optimizer, its
    state slots, step counter and learning rate) into existing device tensors."""
    for k, t in params.items():
        if k not in ckpt.initializers:
            raise KeyError(f"parameter {k!r} is not in the checkpoint")
        vals = ckpt.initializers[k]
        if tuple(vals.shape) != tuple(t.shape()):
            raise ValueError(f"parameter {k!r}: checkpoint shape {vals.shape}, tensor {t.shape()}")
        DeviceArray(t.ctx, t.device_ptrs()[0], vals.shape, owned=False).upload(vals)
    if optimizer is None:
        return
    variant, _, slot_names = optimizer._ckpt
    if variant not in ckpt.optimizer:
        raise ValueError(f"checkpoint optimizer {list(ckpt.optimizer)} is not {variant}")
    optimizer.set_learning_rate(ckpt.optimizer[variant]["learning_rate"])
    n, slots, _ = optimizer.state_info()
    for i in range(n):
        pname = _name_of(params, optimizer._params[i])
        for s in range(slots):
            key = f"{pname}.{slot_names[s]}"
            if key in ckpt.optimizer_state:
                optimizer.set_state(i, s, ckpt.optimizer_state[key])
    if "step" in ckpt.optimizer_state:
        optimizer.set_step(int(ckpt.optimizer_state["step"][0]))
