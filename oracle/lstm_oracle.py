"""C5 (2-layer LSTM forecaster) forward and BPTT in float64 numpy -- test
infrastructure.  numrs has no recurrent layer, so this is the mathematics
(gate order i, f, g, o, one bias per layer), pinned against torch float64
autograd in tests/test_oracle_new_ops.py."""
from __future__ import annotations

import math

import numpy as np

from workloads import make_c5  # noqa: F401  (re-exported for the tests)


def _sig(z):
    return 1.0 / (1.0 + np.exp(-z))


def lstm_layer(x, w_ih, w_hh, b):
    """x [B, T, I] float64 -> (h_seq, cache)."""
    B, T, _ = x.shape
    H = w_hh.shape[1]
    h = np.zeros((B, H), x.dtype)
    c = np.zeros((B, H), x.dtype)
    hs, cs, acts = [], [], []
    for t in range(T):
        z = x[:, t] @ w_ih.T + h @ w_hh.T + b
        i, f, g, o = _sig(z[:, :H]), _sig(z[:, H:2 * H]), np.tanh(z[:, 2 * H:3 * H]), _sig(z[:, 3 * H:])
        c = f * c + i * g
        h = o * np.tanh(c)
        hs.append(h)
        cs.append(c)
        acts.append((i, f, g, o))
    return np.stack(hs, 1), (np.stack(cs, 1), acts)


def lstm_layer_backward(x, w_ih, w_hh, h_seq, cache, dh_seq):
    B, T, _ = x.shape
    H = w_hh.shape[1]
    c_seq, acts = cache
    dx = np.zeros_like(x)
    dt = x.dtype
    dwi, dwh, db = np.zeros_like(w_ih), np.zeros_like(w_hh), np.zeros(4 * H, dt)
    dh_next = np.zeros((B, H), dt)
    dc_next = np.zeros((B, H), dt)
    for t in range(T - 1, -1, -1):
        i, f, g, o = acts[t]
        c = c_seq[:, t]
        cp = c_seq[:, t - 1] if t > 0 else np.zeros((B, H), dt)
        hp = h_seq[:, t - 1] if t > 0 else np.zeros((B, H), dt)
        dh = dh_seq[:, t] + dh_next
        tc = np.tanh(c)
        dc = dh * o * (1 - tc ** 2) + dc_next
        dz = np.concatenate([dc * g * i * (1 - i), dc * cp * f * (1 - f), dc * i * (1 - g ** 2),
                             dh * tc * o * (1 - o)], 1)
        dwi += dz.T @ x[:, t]
        dwh += dz.T @ hp
        db += dz.sum(0)
        dx[:, t] = dz @ w_ih
        dh_next = dz @ w_hh
        dc_next = dc * f
    return dx, dwi, dwh, db


def forecaster(layers, head_w, head_b, x, target, dtype=np.float64):
    """Loss and gradients of every parameter (and of x), computed in `dtype`:
    float64 is the oracle; float32 runs the same BPTT in fp32 on the CPU, the
    error scale an fp32 CPU implementation reaches."""
    h = x.astype(dtype)
    ins, outs, caches = [], [], []
    for l in layers:
        w = {k: v.astype(dtype) for k, v in l.items()}
        ins.append(h)
        h, cache = lstm_layer(h, w["w_ih"], w["w_hh"], w["b"])
        outs.append(h)
        caches.append((w, cache))
    last = h[:, -1]
    hw = head_w.astype(dtype)
    y = last @ hw.T + head_b.astype(dtype)
    n = y.size
    target = target.astype(dtype)
    loss = ((y - target) ** 2).sum() / n
    dy = 2 * (y - target) / n
    grads = {"head_w": dy.T @ last, "head_b": dy.sum(0)}
    dh = np.zeros_like(h)
    dh[:, -1] = dy @ hw
    for li in range(len(layers) - 1, -1, -1):
        w, cache = caches[li]
        dxl, dwi, dwh, db = lstm_layer_backward(ins[li], w["w_ih"], w["w_hh"], outs[li], cache, dh)
        grads[f"w_ih{li}"], grads[f"w_hh{li}"], grads[f"b{li}"] = dwi, dwh, db
        dh = dxl
    grads["x"] = dh
    return loss, grads, y
