"""C1 (2-layer MLP) train step composed from the CPU oracle, in the node order
numrs records it -- test infrastructure.

Forward (autograd/nn.rs:217-235, ops.rs): for each Linear, Transpose(W) ->
MatMul(x, W^T) -> Add(., b); ReLU between; cross_entropy_loss at the end.
Backward walks those nodes in reverse (tensor.rs:173-215):
cross_entropy_backward -> add_backward (+ unbroadcast of the bias) ->
matmul_backward -> transpose_backward -> relu_backward -> ... .  SGD then
updates every parameter (optim/sgd.rs:87-124).

The forward products use the float64 oracle (the reference's forward sgemm is
MKL, not vendored: its bits are not reproducible); everything in-tree Rust is
restated faithfully.
"""
from __future__ import annotations

import numpy as np

from oracle import oracle as O
from workloads import make_c1, xavier  # noqa: F401  (re-exported for the tests)


def _bias_grad(g, n, mode):
    if mode == "correct":
        return O.sum_to_shape(g, (n,))
    out = np.zeros(n, np.float32)
    O.unbroadcast_reference_accumulate(g, out)
    return out


def mlp_step(p: dict, lr: float = 0.01, mode: str = "correct"):
    """One forward + backward + SGD step; returns (loss, grads, new params)."""
    x, labels = p["x"], p["labels"]
    onehot = np.eye(p["W2"].shape[0], dtype=np.float32)[labels]
    W1t = O.transpose(p["W1"])
    z1 = O.matmul_f64(x, W1t) + p["b1"]
    h = O.relu(z1)
    W2t = O.transpose(p["W2"])
    z2 = O.matmul_f64(h, W2t) + p["b2"]
    loss = O.cross_entropy_loss(z2, onehot)

    dz2 = O.cross_entropy_backward(1.0, z2, onehot)
    db2 = _bias_grad(dz2, p["b2"].size, mode)
    dh, dW2t = O.matmul_backward(dz2, h, W2t, f64=True)
    dW2 = O.transpose(dW2t)
    dz1 = O.relu_backward(dh, z1)
    db1 = _bias_grad(dz1, p["b1"].size, mode)
    _, dW1t = O.matmul_backward(dz1, x, W1t, need_a=False, f64=True)
    dW1 = O.transpose(dW1t)
    grads = {"W1": dW1, "b1": db1, "W2": dW2, "b2": db2}

    new = {k: v.copy() for k, v in p.items()}
    for k in ("W1", "b1", "W2", "b2"):
        O.sgd_step(new[k], grads[k], None, lr)
    return loss, grads, new
