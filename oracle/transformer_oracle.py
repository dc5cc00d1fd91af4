"""C4 (pre-LN transformer encoder block) forward and backward in float64
numpy -- test infrastructure.  The block has no numrs counterpart (no
attention, LayerNorm or GELU in the reference), so this is the mathematics:
closed-form backward of every node, pinned against torch float64 autograd in
tests/test_oracle_new_ops.py.  LayerNorm / GELU / softmax backward reuse the
C oracle's float64 routines where they exist.
"""
from __future__ import annotations

import math

import numpy as np

from workloads import make_c4  # noqa: F401  (re-exported for the tests)


def _ln(x, eps=1e-5):
    mu = x.mean(1, keepdims=True)
    var = ((x - mu) ** 2).mean(1, keepdims=True)
    rs = 1.0 / np.sqrt(var + eps)
    return (x - mu) * rs, rs


def _ln_bwd(g, xh, rs, gamma):
    gg = g * gamma
    return rs * (gg - gg.mean(1, keepdims=True) - xh * (gg * xh).mean(1, keepdims=True))


try:
    from scipy.special import erf as _erf
except ImportError:  # pragma: no cover
    _erf = np.vectorize(math.erf)


def _gelu(x):
    return x * 0.5 * (1.0 + _erf(x / math.sqrt(2.0)))


def _gelu_grad(x):
    return 0.5 * (1.0 + _erf(x / math.sqrt(2.0))) + x * np.exp(-0.5 * x * x) / math.sqrt(2 * math.pi)


def _heads(a, B, S, H):
    return a.reshape(B, S, H, -1).transpose(0, 2, 1, 3)  # [B, H, S, dh]


def _merge(a, B, S):
    return a.transpose(0, 2, 1, 3).reshape(B * S, -1)


def attention_forward(q, k, v, B, S, H):
    """softmax(Q K^T / sqrt(dh)) V per head; q, k, v [B*S, H*dh] float64.
    Returns the merged output [B*S, H*dh] and what the backward needs."""
    dh = q.shape[1] // H
    Q, K, V = _heads(q, B, S, H), _heads(k, B, S, H), _heads(v, B, S, H)
    s = Q @ K.transpose(0, 1, 3, 2) / math.sqrt(dh)
    s = s - s.max(-1, keepdims=True)
    P = np.exp(s)
    P /= P.sum(-1, keepdims=True)
    return _merge(P @ V, B, S), (Q, K, V, P, dh)


def attention_backward(dA, cache, B, S, H):
    """Grads of q, k, v [B*S, H*dh] from the merged output grad dA."""
    Q, K, V, P, dh = cache
    dA = _heads(dA, B, S, H)
    dV = P.transpose(0, 1, 3, 2) @ dA
    dP = dA @ V.transpose(0, 1, 3, 2)
    dS = P * (dP - (dP * P).sum(-1, keepdims=True)) / math.sqrt(dh)
    dQ, dK = dS @ K, dS.transpose(0, 1, 3, 2) @ Q
    return _merge(dQ, B, S), _merge(dK, B, S), _merge(dV, B, S)


def block(w, x, t, dims, dtype=np.float64):
    """Returns (loss, grads dict, output y), computed in `dtype`: float64 is
    the oracle; float32 runs the same chain in fp32 on the CPU (BLAS sgemm
    products), the error scale an fp32 CPU implementation reaches."""
    B, S, H = dims
    f = {k: v.astype(dtype) for k, v in w.items()}
    x = x.astype(dtype)
    t = t.astype(dtype)
    xh1, rs1 = _ln(x)
    ln1 = xh1  # gamma 1, beta 0
    q, k, v = ln1 @ f["wq"].T, ln1 @ f["wk"].T, ln1 @ f["wv"].T
    A, att = attention_forward(q, k, v, B, S, H)
    o = A @ f["wo"].T
    r = x + o
    xh2, rs2 = _ln(r)
    h1 = xh2 @ f["w1"].T
    a1 = _gelu(h1)
    y = r + a1 @ f["w2"].T
    n = y.size
    loss = ((y - t) ** 2).sum() / n

    dy = 2.0 * (y - t) / n
    g = {}
    g["w2"] = dy.T @ a1
    da1 = dy @ f["w2"]
    dh1 = da1 * _gelu_grad(h1)
    g["w1"] = dh1.T @ xh2
    dln2 = dh1 @ f["w1"]
    g["ln2_gamma"] = (dln2 * xh2).sum(0)
    g["ln2_beta"] = dln2.sum(0)
    dr = dy + _ln_bwd(dln2, xh2, rs2, 1.0)
    g["wo"] = dr.T @ A
    dq, dk, dv = attention_backward(dr @ f["wo"], att, B, S, H)
    g["wq"], g["wk"], g["wv"] = dq.T @ ln1, dk.T @ ln1, dv.T @ ln1
    dln1 = dq @ f["wq"] + dk @ f["wk"] + dv @ f["wv"]
    g["ln1_gamma"] = (dln1 * xh1).sum(0)
    g["ln1_beta"] = dln1.sum(0)
    g["x"] = dr + _ln_bwd(dln1, xh1, rs1, 1.0)
    g["bq"], g["bk"], g["bv"] = dq.sum(0), dk.sum(0), dv.sum(0)
    g["bo"], g["c1"], g["c2"] = dr.sum(0), dh1.sum(0), dy.sum(0)
    return loss, g, y
