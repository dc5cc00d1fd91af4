"""NN modules over the device Tensor (mirrors numrs-core/src/autograd/nn.rs).

`Linear.forward` records the reference's node sequence exactly --
Transpose(W), MatMul(x, W^T), Add(., b) (nn.rs:217-235) -- so its backward
runs transpose_backward, matmul_backward and add_backward/unbroadcast.
"""
from __future__ import annotations

import numpy as np

from .autograd import Tensor, default_context


class Module:
    """trait Module (nn.rs:23-42)."""

    training = True

    def forward(self, x: Tensor) -> Tensor:
        raise NotImplementedError

    def __call__(self, x: Tensor) -> Tensor:
        return self.forward(x)

    def parameters(self) -> list[Tensor]:
        return []

    def train(self) -> None:
        self.training = True

    def eval(self) -> None:
        self.training = False


class Linear(Module):
    """y = x @ W^T + b with W [out, in], b [out] (nn.rs:57-235).

    By default the layer is one fused node (an NT product with the bias in its
    epilogue; backward dx = g W and dW = g^T x in one launch).  `fused=False`
    records the reference's own three nodes instead; both give the same
    gradients."""

    fused = True

    def __init__(self, in_features: int, out_features: int, ctx=None):
        # Linear::new's deterministic fill: sin(0.123 i) * sqrt(1/in) (nn.rs:67-96).
        k = np.float32(np.sqrt(np.float32(1.0) / np.float32(in_features)))
        i = np.arange(in_features * out_features, dtype=np.float32)
        w = (np.sin(i * np.float32(0.123)) * k).astype(np.float32)
        self._init(in_features, out_features, w, np.zeros(out_features, np.float32), ctx)

    @classmethod
    def with_weights(cls, in_features: int, out_features: int, weight, bias, ctx=None) -> "Linear":
        """Linear::with_weights (nn.rs:107-129)."""
        obj = cls.__new__(cls)
        obj._init(in_features, out_features, weight, bias, ctx)
        return obj

    def _init(self, fin, fout, w, b, ctx):
        ctx = ctx or default_context()
        self.in_features, self.out_features = fin, fout
        self.weight = Tensor.new(np.asarray(w, np.float32).reshape(fout, fin), True, ctx=ctx)
        self.bias = Tensor.new(np.asarray(b, np.float32).reshape(fout), True, ctx=ctx)

    def forward(self, x: Tensor) -> Tensor:
        if self.fused:
            return x.linear(self.weight, self.bias)
        w_t = self.weight.transpose()
        return x.matmul(w_t).add(self.bias)

    def parameters(self) -> list[Tensor]:
        return [self.weight, self.bias]


class ReLU(Module):
    def forward(self, x: Tensor) -> Tensor:  # nn.rs:306-320
        return x.relu()


class Sigmoid(Module):
    def forward(self, x: Tensor) -> Tensor:  # nn.rs:324-338
        return x.sigmoid()


class Tanh(Module):
    def forward(self, x: Tensor) -> Tensor:
        return x.tanh()


class GELU(Module):
    def forward(self, x: Tensor) -> Tensor:
        return x.gelu()


class Softmax(Module):
    """Row softmax over the last axis (nn.rs:345-375 asks for it; the
    reference's ops::softmax cannot take an axis)."""

    def forward(self, x: Tensor) -> Tensor:
        return x.softmax()


class LayerNorm(Module):
    def __init__(self, features: int, eps: float = 1e-5, ctx=None):
        ctx = ctx or default_context()
        self.eps = eps
        self.gamma = Tensor.new(np.ones(features, np.float32), True, ctx=ctx)
        self.beta = Tensor.new(np.zeros(features, np.float32), True, ctx=ctx)

    def forward(self, x: Tensor) -> Tensor:
        return x.layer_norm(self.gamma, self.beta, self.eps)

    def parameters(self) -> list[Tensor]:
        return [self.gamma, self.beta]


class Sequential(Module):
    """nn.rs:257-302.

    A fused Linear directly followed by ReLU runs as one Linear+ReLU node
    (`fuse_relu`, default on): the same output and parameter gradients, one
    node fewer (the pre-activation is not a tensor of its own)."""

    fuse_relu = True

    def __init__(self, layers):
        self.layers = list(layers)

    def add(self, layer: Module) -> None:
        self.layers.append(layer)

    def forward(self, x: Tensor) -> Tensor:
        i, layers = 0, self.layers
        while i < len(layers):
            layer = layers[i]
            if (self.fuse_relu and type(layer) is Linear and layer.fused and i + 1 < len(layers)
                    and type(layers[i + 1]) is ReLU):
                x = x.linear(layer.weight, layer.bias, relu=True)
                i += 2
                continue
            x = layer.forward(x)
            i += 1
        return x

    def parameters(self) -> list[Tensor]:
        return [p for layer in self.layers for p in layer.parameters()]

    def train(self) -> None:
        for layer in self.layers:
            layer.train()

    def eval(self) -> None:
        for layer in self.layers:
            layer.eval()


class MultiHeadAttention(Module):
    """Self-attention projections + fused attention node (no reference op).

    By default (`fused_qkv`) the q, k and v projections are one Linear to 3d
    features, W_qkv = [W_q; W_k; W_v] and b_qkv = [b_q; b_k; b_v], whose packed
    [batch*seq, 3d] output the attention node reads in place: one product
    forward and one product pair backward instead of three.  `fused_qkv =
    False` keeps three Linear layers; both give the same values and grads.
    The choice is made per instance at construction (the class attribute is
    only the default) and fixes the parameter layout: parameters() is
    [W_qkv, b_qkv, W_o, b_o] packed, or [W_q, b_q, W_k, b_k, W_v, b_v, W_o,
    b_o] unpacked, which an optimizer's state and a checkpoint follow."""

    fused_qkv = True

    def __init__(self, wq, wk, wv, wo, heads: int, ctx=None, fused_qkv: bool | None = None):
        d = np.asarray(wq).shape[0]
        z = np.zeros(d, np.float32)
        self.heads, self.dim = heads, d
        self._fused_qkv = type(self).fused_qkv if fused_qkv is None else bool(fused_qkv)
        if self._fused_qkv:
            w = np.concatenate([np.asarray(a, np.float32).reshape(d, d) for a in (wq, wk, wv)])
            self.qkv = Linear.with_weights(d, 3 * d, w, np.zeros(3 * d, np.float32), ctx)
            self.projections = [self.qkv]
        else:
            self.q = Linear.with_weights(d, d, wq, z, ctx)
            self.k = Linear.with_weights(d, d, wk, z, ctx)
            self.v = Linear.with_weights(d, d, wv, z, ctx)
            self.projections = [self.q, self.k, self.v]
        self.o = Linear.with_weights(d, d, wo, z, ctx)

    def forward_seq(self, x: Tensor, batch: int, seq: int, residual: Tensor | None = None
                    ) -> Tensor:
        """Attention output projection of x [batch*seq, d]; with `residual`,
        residual + that projection (one node when the projection is a fused
        Linear)."""
        if self._fused_qkv:
            a = self.qkv(x).attention_qkv(batch, seq, self.heads)
        else:
            a = self.q(x).attention(self.k(x), self.v(x), batch, seq, self.heads)
        if residual is None:
            return self.o(a)
        if self.o.fused:
            return a.linear(self.o.weight, self.o.bias, residual=residual)
        return residual.add(self.o(a))

    def projection_grads(self) -> dict:
        """Gradients of the q, k, v projections as wq, wk, wv [d, d] and bq,
        bk, bv [d], from either form."""
        d = self.dim
        if not self._fused_qkv:
            out = {f"w{n}": getattr(self, n).weight.gradient() for n in ("q", "k", "v")}
            out.update({f"b{n}": getattr(self, n).bias.gradient() for n in ("q", "k", "v")})
            return out
        gw, gb = self.qkv.weight.gradient(), self.qkv.bias.gradient()
        out = {}
        for i, n in enumerate(("q", "k", "v")):
            out[f"w{n}"] = gw[i * d:(i + 1) * d]
            out[f"b{n}"] = gb[i * d:(i + 1) * d]
        return out

    def parameters(self) -> list[Tensor]:
        return [p for m in self.projections + [self.o] for p in m.parameters()]


class TransformerEncoderBlock(Module):
    """Pre-LN encoder block on x [batch*seq, d_model]:
    r = x + Attn(LN1(x));  y = r + W2 GELU(W1 LN2(r)).

    With `fuse_residual` (default) each residual add rides in the epilogue of
    the projection before it (one node each, same values and gradients)."""

    fuse_residual = True

    def __init__(self, weights: dict, heads: int, ctx=None):
        d = np.asarray(weights["wq"]).shape[0]
        f = np.asarray(weights["w1"]).shape[0]
        self.ln1 = LayerNorm(d, ctx=ctx)
        self.ln2 = LayerNorm(d, ctx=ctx)
        self.attn = MultiHeadAttention(weights["wq"], weights["wk"], weights["wv"], weights["wo"],
                                       heads, ctx)
        self.ff1 = Linear.with_weights(d, f, weights["w1"], np.zeros(f, np.float32), ctx)
        self.ff2 = Linear.with_weights(f, d, weights["w2"], np.zeros(d, np.float32), ctx)

    def forward_seq(self, x: Tensor, batch: int, seq: int) -> Tensor:
        if not (self.fuse_residual and self.ff1.fused and self.ff2.fused):
            r = x.add(self.attn.forward_seq(self.ln1(x), batch, seq))
            return r.add(self.ff2(self.ff1(self.ln2(r)).gelu()))
        r = self.attn.forward_seq(self.ln1(x), batch, seq, residual=x)
        # GELU stays a node of its own: in the FFN's first projection the
        # epilogue would also store the pre-activation, and that 256 x 128
        # tile epilogue (every CU writing at once) costs more than the
        # separate pass (measured on MI355X at [4096, 2048]).
        h = self.ff1(self.ln2(r)).gelu()
        return h.linear(self.ff2.weight, self.ff2.bias, residual=r)

    def parameters(self) -> list[Tensor]:
        return (self.ln1.parameters() + self.attn.parameters() + self.ln2.parameters() +
                self.ff1.parameters() + self.ff2.parameters())


class LSTM(Module):
    """One LSTM layer (gate order i, f, g, o) over x [B, T, I] -> [B, T, H]."""

    def __init__(self, w_ih, w_hh, bias=None, ctx=None):
        w_ih = np.asarray(w_ih, np.float32)
        w_hh = np.asarray(w_hh, np.float32)
        self.hidden = w_hh.shape[1]
        self.w_ih = Tensor.new(w_ih, True, ctx=ctx)
        self.w_hh = Tensor.new(w_hh, True, ctx=ctx)
        b = np.zeros(4 * self.hidden, np.float32) if bias is None else bias
        self.bias = Tensor.new(np.asarray(b, np.float32), True, ctx=ctx)

    def forward(self, x: Tensor) -> Tensor:
        return x.lstm(self.w_ih, self.w_hh, self.bias)

    def parameters(self) -> list[Tensor]:
        return [self.w_ih, self.w_hh, self.bias]


class LSTMForecaster(Module):
    """Stacked LSTM layers and a Linear head on the last step's hidden state.

    Two layers run as one stacked node (`fuse_stack`, default on): the
    layers' steps interleave, layer 1's step t beside layer 2's step t - 1
    in one launch; the same values and gradients as two layer nodes up to
    fp32 rounding order."""

    fuse_stack = True

    def __init__(self, layers: list[dict], head_w, head_b, ctx=None):
        self.layers = [LSTM(l["w_ih"], l["w_hh"], l.get("b"), ctx) for l in layers]
        hw = np.asarray(head_w, np.float32)
        self.head = Linear.with_weights(hw.shape[1], hw.shape[0], hw, head_b, ctx)

    def forward(self, x: Tensor) -> Tensor:
        if self.fuse_stack and len(self.layers) == 2:
            a, b = self.layers
            x = x.lstm2(a.w_ih, a.w_hh, a.bias, b.w_ih, b.w_hh, b.bias)
        else:
            for layer in self.layers:
                x = layer.forward(x)
        return self.head(x.time_slice(x.shape()[1] - 1))

    def parameters(self) -> list[Tensor]:
        return [p for l in self.layers for p in l.parameters()] + self.head.parameters()
