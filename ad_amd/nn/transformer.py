"""Post-norm transformer encoder (autodiff/nn/transformer.py).

Attention scores are scaled by 1/sqrt(d_model) (not by the head width) and
the softmax subtracts no maximum, as in the reference; the per-head
projections are bias-free Linears to d_model / num_heads columns.  Parameter
creation order (all query projections, then keys, values, the output
projection; the two norms before the feed-forward) fixes the Tensor ids."""
from math import sqrt
from typing import Optional

from .linear import Linear
from .module import Module
from .normalization import LayerNorm
from .sequential import Sequential

__all__ = ["Attention", "MultiHeadAttention", "AttentionFeedforward",
           "TransformerEncoderLayer", "TransformerEncoder"]


def scaled_attention(q, k, v, d_model: int, mask=None):
    """softmax(q k^T / sqrt(d_model)) v, with ``mask`` multiplied into the
    scores when given."""
    from .. import dot
    scores = dot(q, k.T()) / sqrt(float(d_model))
    if mask is not None:
        scores = scores * mask
    return dot(scores.softmax(-1), v)


class Attention(Module):
    def forward(self, Q, K, V, d_model: int, mask=None):
        return scaled_attention(Q, K, V, d_model, mask)


def _projections(d_in: int, d_out: int, count: int):
    return [Linear(d_in, d_out, bias=False) for _ in range(count)]


class MultiHeadAttention(Module):
    def __init__(self, d_model: int, num_heads: int):
        super().__init__()
        if d_model % num_heads:
            raise AssertionError(f"{num_heads} heads do not divide d_model {d_model}")
        width = d_model // num_heads
        self.wq = _projections(d_model, width, num_heads)
        self.wk = _projections(d_model, width, num_heads)
        self.wv = _projections(d_model, width, num_heads)
        self.attentions = [Attention() for _ in range(num_heads)]
        self.wo = Linear(d_model, d_model, bias=False)
        self.num_heads = num_heads
        self.d_model = d_model

    def head(self, i: int, Q, K, V, mask=None):
        """Head ``i``: its projections of Q, K and V, then attention."""
        return self.attentions[i](self.wq[i](Q), self.wk[i](K), self.wv[i](V), self.d_model, mask)

    def forward(self, Q, K, V, mask: Optional[object] = None):
        from .. import concat
        heads = [self.head(i, Q, K, V, mask) for i in range(self.num_heads)]
        return self.wo(concat(heads, -1))


class AttentionFeedforward(Module):
    """relu(x W1 + b1) W2 + b2."""

    def __init__(self, d_model: int, inner_dim: int):
        super().__init__()
        self.f_expand = Linear(d_model, inner_dim)
        self.f_contract = Linear(inner_dim, d_model)

    def forward(self, x):
        hidden = self.f_expand(x).relu()
        return self.f_contract(hidden)


class TransformerEncoderLayer(Module):
    """y = LN(x + MHA(x, x, x)); out = LN(y + FFN(y))."""

    def __init__(self, d_model: int, num_heads: int, ff_dim: int):
        super().__init__()
        self.attention = MultiHeadAttention(d_model, num_heads)
        self.layer_norm_att = LayerNorm(d_model)
        self.layer_norm_ffwd = LayerNorm(d_model)
        self.ffwd = AttentionFeedforward(d_model, ff_dim)

    def forward(self, x):
        mixed = self.layer_norm_att(x + self.attention(x, x, x))
        return self.layer_norm_ffwd(mixed + self.ffwd(mixed))


class TransformerEncoder(Module):
    def __init__(self, num_layers: int, d_model: int, num_heads: int, ff_dim: int):
        super().__init__()
        self.seq = Sequential(*[TransformerEncoderLayer(d_model, num_heads, ff_dim) for _ in range(num_layers)])

    def forward(self, x):
        return self.seq(x)
