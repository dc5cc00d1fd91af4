"""Writes the golden fixtures of the autograd hot path (tests/golden/*.npz).

    python tests/golden/make_golden.py

Every expected output comes from torch autograd in float64 on the CPU, fed
the float32 inputs stored beside it, so the fixtures are independent of both
the C oracle and the HIP kernels.  Where numrs's semantics and torch's
agree, the fixtures pin them:

* matmul grads dA = dC.B^T, dB = A^T.dC       (backward.rs:113-149)
* unary grads with numrs's strict x > 0 ReLU mask  (backward.rs:152-205,
  407-517); GELU in its exact erf form (new op)
* add/sub/mul/div grads with a broadcast bias row reduced over the rows
  (backward.rs:43-109; the column reduction, not the reference's full sum)
* sum/mean grads (backward.rs:208-236), MSE (backward.rs:239-261, mean over
  all elements), softmax cross-entropy with a batch mean
  (backward.rs:265-301), row softmax backward (backward.rs:521-541)
* LayerNorm, attention and LSTM grads (new ops; LSTM gate order i, f, g, o,
  one bias per layer, x [B, T, I])
* argmax over rows with ties, first and last maximum
  (scalar.rs:517-528, train.rs:213-228)
* SGD with momentum and weight decay, and Adam, over three steps
  (optim/sgd.rs:87-124, optim/adam.rs:124-167)
* one full C1 step: x[64,784], Linear 784->128, ReLU, Linear 128->10,
  cross-entropy against integer labels

Only test code reads the fixtures (numpy.load, no pickles).
"""
from __future__ import annotations

import math
import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
SEED = 20261202


def _t(a, grad=False):
    return torch.tensor(np.asarray(a, np.float64), dtype=torch.float64, requires_grad=grad)


def _n(t):
    return t.detach().numpy().astype(np.float64)


def grads_small(rng) -> dict:
    out = {}
    f32 = lambda a: np.asarray(a, np.float32)  # noqa: E731

    # matmul C[6,7] = A[6,5] B[5,7], upstream G
    A, B, G = f32(rng.standard_normal((6, 5))), f32(rng.standard_normal((5, 7))), f32(
        rng.standard_normal((6, 7)))
    ta, tb = _t(A, True), _t(B, True)
    (ta @ tb).backward(_t(G))
    out.update(mm_A=A, mm_B=B, mm_G=G, mm_dA=_n(ta.grad), mm_dB=_n(tb.grad))

    # unary grads on 96 points; x[0] = 0 (ReLU mask), x[1] = -0.0
    x = f32(rng.standard_normal(96) * 1.5)
    x[0], x[1] = 0.0, -0.0
    g = f32(rng.standard_normal(96))
    xp = f32(np.abs(x) + 0.25)  # log, sqrt domain
    xt = f32(np.clip(x, -1.2, 1.2))  # tan away from its poles
    out.update(un_x=x, un_xp=xp, un_xt=xt, un_g=g)
    fns = {
        "relu": (x, torch.relu), "sigmoid": (x, torch.sigmoid), "tanh": (x, torch.tanh),
        "exp": (x, torch.exp), "log": (xp, torch.log), "sqrt": (xp, torch.sqrt),
        "sin": (x, torch.sin), "cos": (x, torch.cos), "tan": (xt, torch.tan),
        "pow3": (x, lambda v: v ** 3), "gelu": (x, lambda v: F.gelu(v, approximate="none")),
    }
    for name, (inp, fn) in fns.items():
        tx = _t(inp, True)
        y = fn(tx)
        y.backward(_t(g))
        out[f"un_{name}_y"] = _n(y)
        out[f"un_{name}_dx"] = _n(tx.grad)

    # binary ops X[5,6] (op) b[6], b broadcast over the rows
    X = f32(rng.standard_normal((5, 6)))
    b = f32(rng.uniform(0.5, 2.0, 6) * np.sign(rng.standard_normal(6)))
    Gb = f32(rng.standard_normal((5, 6)))
    out.update(bin_X=X, bin_b=b, bin_G=Gb)
    for name, fn in (("add", torch.add), ("sub", torch.sub), ("mul", torch.mul),
                     ("div", torch.div)):
        tx, tbb = _t(X, True), _t(b, True)
        fn(tx, tbb).backward(_t(Gb))
        out[f"bin_{name}_dX"] = _n(tx.grad)
        out[f"bin_{name}_db"] = _n(tbb.grad)

    # sum / mean of S[4,5]
    S = f32(rng.standard_normal((4, 5)))
    ts = _t(S, True)
    ts.sum().backward()
    out.update(red_S=S, red_sum=np.float64(S.astype(np.float64).sum()), red_sum_dS=_n(ts.grad))
    ts = _t(S, True)
    ts.mean().backward()
    out.update(red_mean=np.float64(S.astype(np.float64).mean()), red_mean_dS=_n(ts.grad))

    # MSE over P[8,3]
    P, T = f32(rng.standard_normal((8, 3))), f32(rng.standard_normal((8, 3)))
    tp = _t(P, True)
    loss = F.mse_loss(tp, _t(T))
    loss.backward()
    out.update(mse_P=P, mse_T=T, mse_loss=_n(loss), mse_dP=_n(tp.grad))

    # softmax cross-entropy, logits[8,10], integer labels
    Lg = f32(rng.standard_normal((8, 10)) * 2.0)
    lab = rng.integers(0, 10, 8).astype(np.int32)
    tl = _t(Lg, True)
    loss = F.cross_entropy(tl, torch.tensor(lab, dtype=torch.int64))
    loss.backward()
    out.update(ce_logits=Lg, ce_labels=lab, ce_loss=_n(loss), ce_dlogits=_n(tl.grad))

    # row softmax and its backward, X[6,9]
    Xs, Gs = f32(rng.standard_normal((6, 9)) * 2.0), f32(rng.standard_normal((6, 9)))
    tx = _t(Xs, True)
    y = torch.softmax(tx, dim=1)
    y.backward(_t(Gs))
    out.update(sm_X=Xs, sm_G=Gs, sm_y=_n(y), sm_dX=_n(tx.grad))

    # LayerNorm over the last axis, X[6,16], eps 1e-5
    Xn = f32(rng.standard_normal((6, 16)) * 1.5 + 0.3)
    gam, bet = f32(rng.uniform(0.5, 1.5, 16)), f32(rng.standard_normal(16) * 0.1)
    Gn = f32(rng.standard_normal((6, 16)))
    tx, tg, tbb = _t(Xn, True), _t(gam, True), _t(bet, True)
    y = F.layer_norm(tx, (16,), tg, tbb, eps=1e-5)
    y.backward(_t(Gn))
    out.update(ln_X=Xn, ln_gamma=gam, ln_beta=bet, ln_G=Gn, ln_y=_n(y), ln_dX=_n(tx.grad),
               ln_dgamma=_n(tg.grad), ln_dbeta=_n(tbb.grad))

    # attention: batch 2, seq 8, heads 2 of 4; q, k, v [batch*seq, heads*dh]
    Bt, Sq, H, dh = 2, 8, 2, 4
    q, k, v = (f32(rng.standard_normal((Bt * Sq, H * dh))) for _ in range(3))
    dO = f32(rng.standard_normal((Bt * Sq, H * dh)))
    tq, tk, tv = _t(q, True), _t(k, True), _t(v, True)

    def heads(t):
        return t.reshape(Bt, Sq, H, dh).permute(0, 2, 1, 3)

    att = torch.softmax(heads(tq) @ heads(tk).transpose(-1, -2) / math.sqrt(dh), dim=-1)
    o = (att @ heads(tv)).permute(0, 2, 1, 3).reshape(Bt * Sq, H * dh)
    o.backward(_t(dO))
    out.update(att_q=q, att_k=k, att_v=v, att_dO=dO, att_shape=np.array([Bt, Sq, H, dh]),
               att_o=_n(o), att_dq=_n(tq.grad), att_dk=_n(tk.grad), att_dv=_n(tv.grad))

    # LSTM layer: x [B=2, T=3, I=4], hidden 5, gates i, f, g, o, one bias
    Bl, Tl, Il, Hl = 2, 3, 4, 5
    xl = f32(rng.standard_normal((Bl, Tl, Il)))
    wih, whh = f32(rng.standard_normal((4 * Hl, Il)) * 0.4), f32(
        rng.standard_normal((4 * Hl, Hl)) * 0.4)
    bl = f32(rng.standard_normal(4 * Hl) * 0.1)
    Gl = f32(rng.standard_normal((Bl, Tl, Hl)))
    lstm = torch.nn.LSTM(Il, Hl, batch_first=True).double()
    with torch.no_grad():
        lstm.weight_ih_l0.copy_(_t(wih))
        lstm.weight_hh_l0.copy_(_t(whh))
        lstm.bias_ih_l0.copy_(_t(bl))
        lstm.bias_hh_l0.zero_()
    tx = _t(xl, True)
    hseq, _ = lstm(tx)
    hseq.backward(_t(Gl))
    out.update(lstm_x=xl, lstm_wih=wih, lstm_whh=whh, lstm_b=bl, lstm_G=Gl, lstm_h=_n(hseq),
               lstm_dx=_n(tx.grad), lstm_dwih=_n(lstm.weight_ih_l0.grad),
               lstm_dwhh=_n(lstm.weight_hh_l0.grad), lstm_db=_n(lstm.bias_ih_l0.grad))

    # argmax over rows with planted ties (first max and last max)
    Xa = f32(rng.integers(-3, 4, (12, 7)))
    first = torch.argmax(_t(Xa), dim=1).numpy()
    last = (Xa.shape[1] - 1) - torch.argmax(_t(Xa[:, ::-1].copy()), dim=1).numpy()
    out.update(am_X=Xa, am_first=first.astype(np.int32), am_last=last.astype(np.int32))

    # SGD (lr 0.1, momentum 0.9, weight decay 0.01) and Adam (lr 0.01) over 3 steps
    p0 = f32(rng.standard_normal(7))
    gs = f32(rng.standard_normal((3, 7)))
    out.update(opt_p0=p0, opt_g=gs)
    for name, mk in (("sgd", lambda ps: torch.optim.SGD(ps, lr=0.1, momentum=0.9,
                                                        weight_decay=0.01)),
                     ("adam", lambda ps: torch.optim.Adam(ps, lr=0.01, betas=(0.9, 0.999),
                                                          eps=1e-8))):
        p = _t(p0, True)
        opt = mk([p])
        traj = []
        for s in range(3):
            p.grad = _t(gs[s])
            opt.step()
            traj.append(_n(p))
        out[f"opt_{name}"] = np.stack(traj)
    return out


def mlp_c1(rng) -> dict:
    """x[64,784] ~ N(0,1), Xavier-uniform weights, zero
    biases, labels uniform in [0, 10); loss and every parameter grad.

    To keep the file small, x and W1 lie on grids that float32 holds exactly
    (x on multiples of 2^-8, W1 on multiples of 2^-14) and are stored as
    int16 with their scale; dW1 is stored as its first 16 rows plus the
    float64 sum of every column (all 128 rows)."""
    def xavier(fout, fin):
        a = math.sqrt(6.0 / (fin + fout))
        return rng.uniform(-a, a, (fout, fin))

    xq = np.clip(np.rint(rng.standard_normal((64, 784)) * 256), -32767, 32767).astype(np.int16)
    W1q = np.rint(xavier(128, 784) * 16384).astype(np.int16)
    x = xq.astype(np.float32) / np.float32(256)
    W1 = W1q.astype(np.float32) / np.float32(16384)
    W2 = xavier(10, 128).astype(np.float32)
    b1, b2 = np.zeros(128, np.float32), np.zeros(10, np.float32)
    lab = rng.integers(0, 10, 64).astype(np.int32)
    tW1, tb1, tW2, tb2 = (_t(a, True) for a in (W1, b1, W2, b2))
    h = torch.relu(_t(x) @ tW1.T + tb1)
    loss = F.cross_entropy(h @ tW2.T + tb2, torch.tensor(lab, dtype=torch.int64))
    loss.backward()
    dW1 = _n(tW1.grad)
    return dict(x_q=xq, x_scale=np.float32(256), W1_q=W1q, W1_scale=np.float32(16384), W2=W2,
                b1=b1, b2=b2, labels=lab, loss=_n(loss), dW1_rows16=dW1[:16],
                dW1_colsum=dW1.sum(0), db1=_n(tb1.grad), dW2=_n(tW2.grad), db2=_n(tb2.grad))


def main() -> None:
    rng = np.random.default_rng(SEED)
    np.savez_compressed(os.path.join(HERE, "grads_small.npz"), **grads_small(rng))
    np.savez_compressed(os.path.join(HERE, "mlp_c1_step.npz"), **mlp_c1(rng))
    for f in ("grads_small.npz", "mlp_c1_step.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
