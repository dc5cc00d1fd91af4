"""Attention (N3) kernels and the C4 transformer block on the GPU against the
float64 oracle (oracle/transformer_oracle.py, pinned to torch autograd)."""
import math

import numpy as np
import pytest

import numrs_amd as nr
from numrs_amd import Tensor, nn
from oracle import transformer_oracle as TO
from tests.conftest import assert_chain, assert_contraction, rand

pytestmark = pytest.mark.gpu


def _mha_ref(q, k, v, B, S, H):
    q, k, v = (a.astype(np.float64) for a in (q, k, v))
    dh = q.shape[1] // H
    Q, K, V = (TO._heads(a, B, S, H) for a in (q, k, v))
    s = Q @ K.transpose(0, 1, 3, 2) / math.sqrt(dh)
    P = np.exp(s - s.max(-1, keepdims=True))
    P /= P.sum(-1, keepdims=True)
    return P, Q, K, V


# (16, 256, 8, 512) is the C4 shape: 128 heads, enough 128 x 64 tiles for the
# batched streamed products (dQ and dK as one pair launch).  Head size 64 with
# S a multiple of 128 (up to 512) takes the fused row-block kernels (Q K^T +
# softmax, dO V^T + softmax backward); S = 128, 384, 512 cover their other
# column-block counts.
@pytest.mark.parametrize("B,S,H,D", [(2, 40, 4, 64), (1, 7, 1, 5), (3, 256, 8, 512),
                                     (16, 256, 8, 512), (2, 128, 2, 128), (1, 384, 1, 64),
                                     (1, 512, 2, 128)])
def test_attention_forward_backward(hip_ctx, B, S, H, D):
    print(f"[gpu] attention B={B} S={S} H={H} D={D}", flush=True)
    rng = np.random.default_rng(B * 1000 + S)
    q, k, v, dO = (rand(rng, (B * S, D)) for _ in range(4))
    c = hip_ctx
    qd, kd, vd, gd = (c.to_device(a) for a in (q, k, v, dO))
    P, out = c.empty((B * H, S, S)), c.empty((B * S, D))
    assert L_attention_fwd(c, qd, kd, vd, P, out, B, S, H, D) == 0
    Pr, Q, K, V = _mha_ref(q, k, v, B, S, H)
    dh = D // H
    assert_contraction(P.numpy().reshape(B, H, S, S), Pr, dh, what="P")
    assert_contraction(out.numpy(), TO._merge(Pr @ V, B, S), S, what="out")
    dq, dk, dv = (c.empty((B * S, D)) for _ in range(3))
    assert L_attention_bwd(c, qd, kd, vd, P, gd, dq, dk, dv, B, S, H, D) == 0
    dA = TO._heads(dO.astype(np.float64), B, S, H)
    dV = Pr.transpose(0, 1, 3, 2) @ dA
    dP = dA @ V.transpose(0, 1, 3, 2)
    dS = Pr * (dP - (dP * Pr).sum(-1, keepdims=True)) / math.sqrt(dh)
    assert_contraction(dv.numpy(), TO._merge(dV, B, S), S, what="dv")
    assert_contraction(dq.numpy(), TO._merge(dS @ K, B, S), S + dh, what="dq")
    assert_contraction(dk.numpy(), TO._merge(dS.transpose(0, 1, 3, 2) @ Q, B, S), S + dh,
                       what="dk")


@pytest.mark.parametrize("B,S,H,D", [(16, 256, 8, 512), (2, 128, 2, 128), (2, 40, 4, 64)])
@pytest.mark.parametrize("acc", [0, 1])
def test_attention_strided_packed_qkv(hip_ctx, B, S, H, D, acc):
    """q, k, v (and dq, dk, dv) as the column blocks of one packed [B*S, 3D]
    buffer (row stride 3D): the fused row-block path (dh = 64, S % 128 == 0)
    and the GEMM fallback, written and accumulated."""
    from numrs_amd import _lib as L
    print(f"[gpu] attention strided B={B} S={S} H={H} D={D} acc={acc}", flush=True)
    rng = np.random.default_rng(3 * B + S)
    qkv, dO, prev = rand(rng, (B * S, 3 * D)), rand(rng, (B * S, D)), rand(rng, (B * S, 3 * D))
    c = hip_ctx
    qd, gd = c.to_device(qkv), c.to_device(dO)
    P, out = c.empty((B * H, S, S)), c.empty((B * S, D))
    f4 = 4  # bytes per float
    lib = L.load()
    assert lib.numrs_hip_attention_forward_strided(
        c.handle, qd.ptr, qd.ptr + D * f4, qd.ptr + 2 * D * f4, 3 * D, P.ptr, out.ptr, D,
        B, S, H, D) == 0
    q, k, v = qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:]
    Pr, Q, K, V = _mha_ref(q, k, v, B, S, H)
    dh = D // H
    assert_contraction(out.numpy(), TO._merge(Pr @ V, B, S), S, what="out")
    dqkv = c.to_device(prev) if acc else c.zeros((B * S, 3 * D))
    assert lib.numrs_hip_attention_backward_strided(
        c.handle, qd.ptr, qd.ptr + D * f4, qd.ptr + 2 * D * f4, 3 * D, P.ptr, gd.ptr, D,
        dqkv.ptr, dqkv.ptr + D * f4, dqkv.ptr + 2 * D * f4, B, S, H, D, acc) == 0
    dA = TO._heads(dO.astype(np.float64), B, S, H)
    dP = dA @ V.transpose(0, 1, 3, 2)
    dS = Pr * (dP - (dP * Pr).sum(-1, keepdims=True)) / math.sqrt(dh)
    ref = np.concatenate([TO._merge(dS @ K, B, S), TO._merge(dS.transpose(0, 1, 3, 2) @ Q, B, S),
                          TO._merge(Pr.transpose(0, 1, 3, 2) @ dA, B, S)], axis=1)
    if acc:
        ref = ref + prev.astype(np.float64)
    assert_contraction(dqkv.numpy(), ref, S + dh, what="dqkv (packed)")


@pytest.mark.parametrize("B,S,H,D", [(16, 256, 8, 512), (3, 256, 8, 512), (2, 128, 2, 128),
                                     (1, 384, 1, 64), (2, 40, 4, 64)])
@pytest.mark.parametrize("acc", [0, 1])
def test_attention_backward_with_output(hip_ctx, B, S, H, D, acc):
    """numrs_hip_attention_backward_out_strided on the packed [B*S, 3D] layout:
    given the forward's output, dh = 64 with S = 256 (two row blocks per head)
    or S = 128 (one) runs the query-row and key-row kernels when nothing
    accumulates; S = 384, S = 40 and acc = 1 take the row-block or GEMM path.
    Each grad against float64, and a second call returns the same bits."""
    from numrs_amd import _lib as L
    print(f"[gpu] attention backward with output B={B} S={S} H={H} D={D} acc={acc}",
          flush=True)
    rng = np.random.default_rng(7 * B + S + acc)
    qkv, dO, prev = rand(rng, (B * S, 3 * D)), rand(rng, (B * S, D)), rand(rng, (B * S, 3 * D))
    c = hip_ctx
    qd, gd = c.to_device(qkv), c.to_device(dO)
    P, out = c.empty((B * H, S, S)), c.empty((B * S, D))
    f4 = 4
    lib = L.load()
    assert lib.numrs_hip_attention_forward_strided(
        c.handle, qd.ptr, qd.ptr + D * f4, qd.ptr + 2 * D * f4, 3 * D, P.ptr, out.ptr, D,
        B, S, H, D) == 0
    q, k, v = qkv[:, :D], qkv[:, D:2 * D], qkv[:, 2 * D:]
    Pr, Q, K, V = _mha_ref(q, k, v, B, S, H)
    dh = D // H
    dA = TO._heads(dO.astype(np.float64), B, S, H)
    dP = dA @ V.transpose(0, 1, 3, 2)
    dS = Pr * (dP - (dP * Pr).sum(-1, keepdims=True)) / math.sqrt(dh)
    ref = np.concatenate([TO._merge(dS @ K, B, S), TO._merge(dS.transpose(0, 1, 3, 2) @ Q, B, S),
                          TO._merge(Pr.transpose(0, 1, 3, 2) @ dA, B, S)], axis=1)
    if acc:
        ref = ref + prev.astype(np.float64)
    got = []
    for _ in range(2):
        dqkv = c.to_device(prev) if acc else c.to_device(np.full((B * S, 3 * D), np.nan, np.float32))
        assert lib.numrs_hip_attention_backward_out_strided(
            c.handle, qd.ptr, qd.ptr + D * f4, qd.ptr + 2 * D * f4, 3 * D, P.ptr, out.ptr, gd.ptr,
            D, dqkv.ptr, dqkv.ptr + D * f4, dqkv.ptr + 2 * D * f4, B, S, H, D, acc) == 0
        got.append(dqkv.numpy())
    for what, sl in (("dq", slice(0, D)), ("dk", slice(D, 2 * D)), ("dv", slice(2 * D, 3 * D))):
        assert_contraction(got[0][:, sl], ref[:, sl], S + dh, what=f"{what} (with output)")
    assert np.array_equal(got[0], got[1]), "two calls differ"


def L_attention_fwd(c, q, k, v, P, out, B, S, H, D):
    from numrs_amd import _lib as L
    return L.load().numrs_hip_attention_forward(c.handle, q.ptr, k.ptr, v.ptr, P.ptr, out.ptr,
                                                B, S, H, D)


def L_attention_bwd(c, q, k, v, P, g, dq, dk, dv, B, S, H, D):
    from numrs_amd import _lib as L
    return L.load().numrs_hip_attention_backward(c.handle, q.ptr, k.ptr, v.ptr, P.ptr, g.ptr,
                                                 dq.ptr, dk.ptr, dv.ptr, B, S, H, D, 0)


def test_gemm_two_level_batch(hip_ctx):
    # C_z = alpha * A_z @ B_z^T over head slices of [B*S, H*dh] (the QK^T product)
    from numrs_amd import _lib as L
    B, S, H, dh = 2, 33, 3, 20
    D = H * dh
    rng = np.random.default_rng(2)
    q, k = rand(rng, (B * S, D)), rand(rng, (B * S, D))
    c = hip_ctx
    out = c.empty((B * H, S, S))
    qd, kd = c.to_device(q), c.to_device(k)
    rc = L.load().numrs_hip_gemm(c.handle, qd.ptr, D, kd.ptr, D, out.ptr, S, S, dh, S, 0, 1, 0.5, 0,
                                 B * H, H, S * D, dh, S * D, dh, H * S * S, S * S)
    assert rc == 0
    Q, K = TO._heads(q.astype(np.float64), B, S, H), TO._heads(k.astype(np.float64), B, S, H)
    ref = 0.5 * (Q @ K.transpose(0, 1, 3, 2))
    assert_contraction(out.numpy().reshape(B, H, S, S), ref, dh)


def _run_block(dims_full, seed):
    w, x, t, dims = TO.make_c4(seed=seed, **dims_full)
    B, S, H = dims
    blk = nn.TransformerEncoderBlock(w, H)
    xt = Tensor.new(x, True)
    y = blk.forward_seq(xt, B, S)
    loss = y.mse_loss(Tensor.new(t, False))
    loss.backward()
    return w, x, t, dims, blk, xt, loss, y


@pytest.mark.parametrize("dims_full", [dict(B=2, S=64, D=128, H=4, F=256),
                                       dict(B=16, S=256, D=512, H=8, F=2048)],
                         ids=["small", "baseline"])
def test_c4_residual_nodes_equal_add_nodes(hip_ctx, dims_full, monkeypatch):
    """The block with each residual add folded into its projection node
    equals the block with separate Add nodes, bit for bit."""
    print(f"[gpu] C4 residual fusion {dims_full}", flush=True)
    nr.set_default_context(hip_ctx)
    out = []
    for fuse in (True, False):
        monkeypatch.setattr(nn.TransformerEncoderBlock, "fuse_residual", fuse)
        w, x, t, dims, blk, xt, loss, y = _run_block(dims_full, seed=6)
        out.append([y.values(), loss.values(), xt.gradient()] +
                    [p.gradient() for p in blk.parameters()])
    for i, (a, b) in enumerate(zip(*out)):
        assert np.array_equal(a, b), i


@pytest.mark.parametrize("fused_qkv", [True, False], ids=["qkv_fused", "qkv_separate"])
@pytest.mark.parametrize("dims_full", [dict(B=2, S=64, D=128, H=4, F=256),
                                       dict(B=16, S=256, D=512, H=8, F=2048)],
                         ids=["small", "baseline"])
def test_c4_block_matches_oracle(hip_ctx, dims_full, fused_qkv, monkeypatch):
    print(f"[gpu] C4 block {dims_full} fused_qkv={fused_qkv}", flush=True)
    nr.set_default_context(hip_ctx)
    monkeypatch.setattr(nn.MultiHeadAttention, "fused_qkv", fused_qkv)
    w, x, t, dims, blk, xt, loss, y = _run_block(dims_full, seed=4)
    ref_loss, g, ref_y = TO.block(w, x, t, dims)
    # The same chain in fp32 on the CPU: the error scale an fp32 CPU
    # implementation reaches, which the GPU must not exceed.
    _, g32, y32 = TO.block(w, x, t, dims, dtype=np.float32)
    assert abs(loss.item() - ref_loss) <= 1e-5 * abs(ref_loss)
    assert_chain(y.values(), ref_y, y32, what="y")
    got = {"wo": blk.attn.o.weight, "w1": blk.ff1.weight, "w2": blk.ff2.weight,
           "ln1_gamma": blk.ln1.gamma, "ln1_beta": blk.ln1.beta, "ln2_gamma": blk.ln2.gamma,
           "ln2_beta": blk.ln2.beta, "bo": blk.attn.o.bias, "c1": blk.ff1.bias,
           "c2": blk.ff2.bias, "x": xt}
    grads = {name: tensor.gradient() for name, tensor in got.items()}
    proj = blk.attn.projection_grads()
    grads.update({n: proj[n] for n in ("wq", "wk", "wv", "bq", "bv")})
    for name, gg in grads.items():
        assert_chain(gg, g[name], g32[name], what=name)
    # The key bias gets no gradient (softmax is shift-invariant along a row):
    # exactly zero in the float64 oracle, rounding noise here.
    assert np.abs(proj["bk"]).max() <= 1e-5 * np.abs(g["bq"]).max() + 1e-12
