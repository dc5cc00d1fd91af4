"""Synthetic inputs of the configs C1, C4 and C5 (seeded numpy
generators; numpy only).  bench.py builds its workloads from these, and the
tests build the same inputs for the oracles.
"""
from __future__ import annotations

import math

import numpy as np


def xavier(rng, fan_out, fan_in):
    a = np.sqrt(6.0 / (fan_in + fan_out))
    return rng.uniform(-a, a, (fan_out, fan_in)).astype(np.float32)


def make_c1(seed: int = 1, batch: int = 64, fin: int = 784, hidden: int = 128, classes: int = 10):
    """BASELINE config 1 inputs: x ~ N(0,1), Xavier-uniform weights, zero
    biases, uniform int labels in [0, classes)."""
    rng = np.random.default_rng(seed)
    return {
        "x": rng.standard_normal((batch, fin), dtype=np.float32),
        "W1": xavier(rng, hidden, fin), "b1": np.zeros(hidden, np.float32),
        "W2": xavier(rng, classes, hidden), "b2": np.zeros(classes, np.float32),
        "labels": rng.integers(0, classes, batch).astype(np.int32),
    }


def make_c4(seed=4, B=16, S=256, D=512, H=8, F=2048):
    """BASELINE config 4 inputs: x, target ~ N(0,1), Xavier-uniform weights,
    LN gamma = 1, beta = 0, zero biases."""
    rng = np.random.default_rng(seed)

    def xav(o, i):
        a = math.sqrt(6.0 / (i + o))
        return rng.uniform(-a, a, (o, i)).astype(np.float32)

    w = {"wq": xav(D, D), "wk": xav(D, D), "wv": xav(D, D), "wo": xav(D, D),
         "w1": xav(F, D), "w2": xav(D, F)}
    x = rng.standard_normal((B * S, D), dtype=np.float32)
    t = rng.standard_normal((B * S, D), dtype=np.float32)
    return w, x, t, (B, S, H)


def _xavier(rng, fan_out, fan_in):
    a = math.sqrt(6.0 / (fan_in + fan_out))
    return rng.uniform(-a, a, (fan_out, fan_in)).astype(np.float32)


def make_c5(seed=5, B=64, T=128, I=64, H=256, n_layers=2):
    """BASELINE config 5 inputs: each feature is a sum of 3 sinusoids with
    random phases plus N(0, 0.1) noise; Xavier-uniform weights, zero biases;
    target ~ N(0, 1) per series (the head predicts one value per series)."""
    rng = np.random.default_rng(seed)
    t = np.arange(T, dtype=np.float64)
    omega = rng.uniform(0.05, 0.5, 3)
    phase = rng.uniform(0.0, 2 * math.pi, (B, I, 3))
    x = np.sin(omega[None, None, None, :] * t[None, :, None, None] + phase[:, None, :, :]).sum(-1)
    x = (x + rng.normal(0.0, 0.1, x.shape)).astype(np.float32)  # [B, T, I]
    layers = []
    fin = I
    for _ in range(n_layers):
        layers.append({"w_ih": _xavier(rng, 4 * H, fin), "w_hh": _xavier(rng, 4 * H, H),
                       "b": np.zeros(4 * H, np.float32)})
        fin = H
    head_w = _xavier(rng, 1, H)
    head_b = np.zeros(1, np.float32)
    target = rng.standard_normal((B, 1)).astype(np.float32)
    return layers, head_w, head_b, x, target
