"""Loaders of the golden fixtures (numpy.load, no pickles); test code only."""
from __future__ import annotations

import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def grads_small() -> dict:
    return dict(np.load(os.path.join(HERE, "grads_small.npz")))


def mlp_c1() -> dict:
    """The C1 fixture with x and W1 restored as float32 (stored as int16 on
    grids that float32 holds exactly)."""
    z = dict(np.load(os.path.join(HERE, "mlp_c1_step.npz")))
    z["x"] = z.pop("x_q").astype(np.float32) / z.pop("x_scale")
    z["W1"] = z.pop("W1_q").astype(np.float32) / z.pop("W1_scale")
    return z
