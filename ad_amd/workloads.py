"""Programs of the benchmark configurations, traced into the global context.

Each builder traces one program; ``ad_amd.compile_proc()`` (or
``ad_amd.execute``) then lowers it.  Seeds: weights 0, inputs 1, upstream
gradients 2 (``np.random.default_rng``).  The same builders feed the parity
tests, the smoke test and ``bench.py``, so every backend sees identical
inputs and weights.

* ``mlp``            -- examples/linear.py:16-46 (Linear-Sigmoid-Linear, SGD).
* ``dotprod_elw``    -- ``sigmoid(A @ B + bias)``: one DotProd+Elw command.
* ``reduce_elw``     -- ``X.sum(-1) * c``: one Reduce+Elw command.
* ``elw_chain``      -- ``((x*0.5 + 1).exp2() + 1).recip() * 3``: one ElwFuse.
* ``layernorm_train``-- LayerNorm fwd+bwd with SGD on gamma/beta
  (autodiff/nn/normalization/layernorm.py:11-15).
* ``transformer``    -- post-norm encoder layers (autodiff/nn/transformer.py:9-85)
  over a batch: the reference has no batched matmul (graph/compute/dotprod.py
  asserts 2-D operands), so per-head projections run on all B*S rows,
  attention runs per sample on ``Index`` slices of those rows, and the
  per-sample outputs are concatenated back along rows, then heads.
"""
from math import sqrt

import numpy as np

from . import concat, ir_for
from .graph import Feeder, Receiver, Tensor
from .nn import SGD, LayerNorm, Linear, Module, Sequential, Sigmoid
from .nn.transformer import Attention

__all__ = ["set_uniform", "mlp", "dotprod_elw", "reduce_elw", "elw_chain", "layernorm_train",
           "BatchedMultiHeadAttention", "BatchedEncoderLayer", "transformer", "TRANSFORMER_CONFIGS",
           "published_transformer"]


def set_uniform(params, seed=0):
    """Overwrite every parameter with U(-1/sqrt(fan_in), 1/sqrt(fan_in)),
    in id order (the reference's N(0,1) init overflows the max-free softmax
    at these widths)."""
    rng = np.random.default_rng(seed)
    for p in sorted(params, key=lambda t: t.id):
        bound = 1.0 / np.sqrt(p.arr.shape[0])
        p.arr[...] = rng.uniform(-bound, bound, p.arr.shape).astype(np.float32)


def mlp(steps=1000, din=255, dh=255, dout=255, rows=2, fill=0.2, receive=True):
    """examples/linear.py: ``Linear(255,255)-Sigmoid-Linear(255,255)``, input
    [2,255] filled 0.2, implicit ``sum`` loss, SGD lr 0.01, ``steps``
    iterations in one ``ir_for``.  Returns a dict filled with the trained
    parameters after execution."""
    net = Sequential(Linear(din, dh), Sigmoid(), Linear(dh, dout))
    set_uniform(net.parameters(), 0)
    opt = SGD(net.parameters(), lr=0.01)
    x = np.full((rows, din), fill, dtype=np.float32)

    def body():
        opt.zero_grad()
        val = Feeder(lambda: x, shape=[rows, din])
        net(val).backward()
        opt.step()
    ir_for(range(steps), body)
    out = {}
    if receive:
        Receiver(lambda *a: out.setdefault("params", [v.copy() for v in a]), opt.parameters)
    return out


def dotprod_elw(M=4096, K=4096, N=4096, seed=1, receive_pre=False):
    """``sigmoid(A @ B + bias)`` with A, B, bias ~ N(0,1).  With
    ``receive_pre`` the pre-activation ``A @ B + bias`` is received as well
    (``out["pre"]``; the same single DotProd+Elw command then also stores
    it), so a check is not blunted by the sigmoid's saturation."""
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((M, K), dtype=np.float32)
    b = rng.standard_normal((K, N), dtype=np.float32)
    bias = rng.standard_normal((N,), dtype=np.float32)
    A, B, C = Tensor(a), Tensor(b), Tensor(bias)
    pre = (A @ B) + C
    r = pre.sigmoid()
    out = {"inputs": (a, b, bias)}
    if receive_pre:
        Receiver(lambda v, p: (out.setdefault("r", v), out.setdefault("pre", p)), [r, pre])
    else:
        Receiver(lambda v: out.setdefault("r", v), [r])
    return out


def reduce_elw(V=8192, R=4096, scale=0.5, seed=1):
    """``X.sum(-1) * scale`` with X ~ N(0,1)."""
    x = np.random.default_rng(seed).standard_normal((V, R), dtype=np.float32)
    r = Tensor(x).sum(-1) * scale
    out = {"inputs": (x,)}
    Receiver(lambda v: out.setdefault("r", v), [r])
    return out


def elw_chain(n=64 << 20, seed=1):
    """Six elementwise ops, one input, one output:
    ``((x*0.5 + 1).exp2() + 1).recip() * 3``."""
    x = np.random.default_rng(seed).standard_normal((n,), dtype=np.float32)
    r = ((Tensor(x) * 0.5 + 1.0).exp2() + 1.0).recip() * 3.0
    out = {"inputs": (x,)}
    Receiver(lambda v: out.setdefault("r", v), [r])
    return out


def layernorm_train(rows=16384, cols=1024, steps=100, lr=0.01, receive=True):
    """LayerNorm fwd+bwd: loss ``sum(LN(x) * dy)`` so dL/dy = dy; SGD on
    gamma/beta keeps the loop body live (dep_opt prunes side-effect-free
    loops).  x, dy ~ N(0,1) (seeds 1, 2); gamma = 1, beta = 0, eps 1e-5."""
    x = Tensor(np.random.default_rng(1).standard_normal((rows, cols), dtype=np.float32))
    dy = Tensor(np.random.default_rng(2).standard_normal((rows, cols), dtype=np.float32))
    ln = LayerNorm(cols)
    opt = SGD(ln.parameters(), lr=lr)

    def body():
        opt.zero_grad()
        (ln(x) * dy).backward()
        opt.step()
    ir_for(range(steps), body)
    out = {}
    if receive:
        Receiver(lambda *a: out.setdefault("params", [v.copy() for v in a]), opt.parameters)
    return out


class BatchedMultiHeadAttention(Module):
    """``MultiHeadAttention`` (autodiff/nn/transformer.py:19-46) over
    ``batch`` sequences of ``seq`` rows stacked in one [batch*seq, d_model]
    matrix.  With ``batch == 1`` the traced graph is the reference's."""

    def __init__(self, d_model, num_heads, batch, seq):
        super().__init__()
        assert d_model % num_heads == 0, "d_model must be divisible by num heads"
        d_v = d_model // num_heads
        self.wq = [Linear(d_model, d_v, bias=False) for _ in range(num_heads)]
        self.wk = [Linear(d_model, d_v, bias=False) for _ in range(num_heads)]
        self.wv = [Linear(d_model, d_v, bias=False) for _ in range(num_heads)]
        self.attentions = [Attention() for _ in range(num_heads)]
        self.wo = Linear(d_model, d_model, bias=False)
        self.num_heads, self.d_model, self.batch, self.seq = num_heads, d_model, batch, seq

    def forward(self, x):
        heads = []
        for i in range(self.num_heads):
            q, k, v = self.wq[i](x), self.wk[i](x), self.wv[i](x)
            if self.batch == 1:
                heads.append(self.attentions[i](q, k, v, self.d_model))
                continue
            per_sample = []
            for b in range(self.batch):
                rows = slice(b * self.seq, (b + 1) * self.seq)
                per_sample.append(self.attentions[i](q[rows], k[rows], v[rows], self.d_model))
            heads.append(concat(per_sample, 0))
        return self.wo(concat(heads, -1))


class BatchedEncoderLayer(Module):
    """``TransformerEncoderLayer`` (autodiff/nn/transformer.py:59-74):
    post-norm attention + ReLU feed-forward."""

    def __init__(self, d_model, num_heads, ff_dim, batch, seq):
        super().__init__()
        from .nn.transformer import AttentionFeedforward
        self.attention = BatchedMultiHeadAttention(d_model, num_heads, batch, seq)
        self.layer_norm_att = LayerNorm(d_model)
        self.layer_norm_ffwd = LayerNorm(d_model)
        self.ffwd = AttentionFeedforward(d_model, ff_dim)

    def forward(self, x):
        y = self.attention(x)
        y = self.layer_norm_att(x + y)
        z = self.ffwd(y)
        return self.layer_norm_ffwd(y + z)


# (layers, d_model, heads, ffn, seq, batch) of the benchmark configurations
TRANSFORMER_CONFIGS = {
    "c4": (1, 512, 8, 2048, 256, 16),
    "c5": (4, 1024, 16, 4096, 512, 8),
}


def transformer(layers=1, d_model=32, heads=4, ff=64, seq=4, batch=1, steps=2, lr=0.01,
                feeder=False, receive=True):
    """Encoder stack fwd + bwd + SGD, MSE-to-zero loss
    ``sum(out*out) / numel`` (the implicit ones-seed of backward, node.py:122,
    makes the loss a sum).  Input X [batch*seq, d_model] ~ N(0,1) (seed 1),
    resident on the device as a Tensor, or fed each step by a Feeder."""
    net = [BatchedEncoderLayer(d_model, heads, ff, batch, seq) for _ in range(layers)]
    params = [p for layer in net for p in layer.parameters()]
    set_uniform(params, 0)
    tensors = list(params)            # SGD.step replaces the entries of ``params``
    opt = SGD(params, lr=lr)
    rows = batch * seq
    x = np.random.default_rng(1).standard_normal((rows, d_model), dtype=np.float32)
    x_t = None if feeder else Tensor(x)

    def body():
        opt.zero_grad()
        out = Feeder(lambda: x, shape=[rows, d_model]) if feeder else x_t
        for layer in net:
            out = layer(out)
        (out * out * (1.0 / (rows * d_model))).backward()
        opt.step()
    ir_for(range(steps), body)
    res = {"params_ref": tensors, "net": net, "x": x}
    if receive:
        Receiver(lambda *a: res.setdefault("params", [v.copy() for v in a]), opt.parameters)
    return res


def published_transformer(layers=1, steps=500, seed=0):
    """examples/transformer.py:13-39, the configuration README.md:34-45 times:
    ``TransformerEncoder(num_layers, d_model=64, num_heads=4, ff_dim=128)``,
    a [2,64] Feeder filled with 0.3 every step, the implicit ``sum`` loss,
    SGD lr 0.01, ``steps`` iterations in one ``ir_for``.  Weights keep the
    reference's N(0,1) ``Linear`` init (seeded here)."""
    from .nn import TransformerEncoder
    np.random.seed(seed)
    net = TransformerEncoder(num_layers=layers, d_model=64, num_heads=4, ff_dim=128)
    opt = SGD(net.parameters(), lr=0.01)
    x = np.full((2, 64), 0.3, dtype=np.float32)

    def body():
        opt.zero_grad()
        net(Feeder(lambda: x, shape=[2, 64])).backward()
        opt.step()
    ir_for(range(steps), body)
    out = {}
    Receiver(lambda *a: out.setdefault("params", len(a)), opt.parameters)
    return out


def dotprod_flops(proc):
    """Algorithmic flops (2*M*N*K) of every DotProd in a Proc, loop bodies
    counted once."""
    from .fusion import DPElwFuse
    from .graph import DotProdNode, ForNode
    total = 0
    for cmd in proc.procedure:
        if isinstance(cmd, ForNode):
            total += dotprod_flops(cmd.get_proc())
            continue
        dp = cmd.init_node if isinstance(cmd, DPElwFuse) else cmd
        if isinstance(dp, DotProdNode):
            M, N = dp.shape
            total += 2 * M * N * dp.children_shapes[0][1]
    return total
