"""Programs traced by the parity tests (the same program is traced twice:
once per backend).  Seeds: weights 0, inputs 1, upstream grads 2."""
import numpy as np

import ad_amd as ad
from ad_amd.graph import Receiver, Tensor
from ad_amd.nn import (SGD, LayerNorm, Linear, Sequential, Sigmoid, TransformerEncoder)


def set_uniform(params, seed):
    rng = np.random.default_rng(seed)
    for p in sorted(params, key=lambda t: t.id):
        bound = 1.0 / np.sqrt(p.arr.shape[0])
        p.arr[...] = rng.uniform(-bound, bound, p.arr.shape).astype(np.float32)


def mlp(steps=3, din=255, dh=255, dout=255, rows=2, fill=0.2):
    """examples/linear.py: Linear-Sigmoid-Linear, implicit sum loss, SGD."""
    net = Sequential(Linear(din, dh), Sigmoid(), Linear(dh, dout))
    set_uniform(net.parameters(), 0)
    opt = SGD(net.parameters(), lr=0.01)

    def body():
        opt.zero_grad()
        val = ad.Feeder(lambda: np.full((rows, din), fill, dtype=np.float32), shape=[rows, din])
        net(val).backward()
        opt.step()
    ad.ir_for(range(steps), body)
    out = {}
    Receiver(lambda *a: out.setdefault("params", [x.copy() for x in a]), opt.parameters)
    return out


def mlp_logged(steps=5, din=16, dh=32, dout=8, rows=4):
    """A small MLP trained in a loop whose body also receives the network's
    output every iteration (per-step logging); returns the outputs in
    callback order and the final parameters."""
    net = Sequential(Linear(din, dh), Sigmoid(), Linear(dh, dout))
    set_uniform(net.parameters(), 0)
    opt = SGD(net.parameters(), lr=0.5)
    x = np.random.default_rng(1).uniform(-1, 1, (rows, din)).astype(np.float32)
    out = {"log": []}

    def body():
        opt.zero_grad()
        val = ad.Feeder(lambda: x, shape=[rows, din])
        y = net(val)
        y.backward()
        opt.step()
        Receiver(lambda v: out["log"].append(v.copy()), [y])
    ad.ir_for(range(steps), body)
    Receiver(lambda *a: out.setdefault("params", [v.copy() for v in a]), opt.parameters)
    return out


def layernorm_step(rows=8, cols=16, steps=2):
    """LayerNorm fwd+bwd with SGD on gamma/beta; loss = sum(LN(x) * dy)."""
    rng = np.random.default_rng(1)
    x = Tensor(rng.standard_normal((rows, cols)).astype(np.float32))
    dy = Tensor(np.random.default_rng(2).standard_normal((rows, cols)).astype(np.float32))
    ln = LayerNorm(cols)
    opt = SGD(ln.parameters(), lr=0.01)

    def body():
        opt.zero_grad()
        (ln(x) * dy).backward()
        opt.step()
    ad.ir_for(range(steps), body)
    out = {}
    Receiver(lambda *a: out.setdefault("params", [v.copy() for v in a]), opt.parameters)
    return out


def transformer(layers=1, d_model=32, heads=4, ff=64, seq=4, steps=2):
    """Transformer encoder on one [seq, d_model] sequence, MSE-to-zero loss."""
    net = TransformerEncoder(num_layers=layers, d_model=d_model, num_heads=heads, ff_dim=ff)
    set_uniform(net.parameters(), 0)
    opt = SGD(net.parameters(), lr=0.01)
    x = np.random.default_rng(1).standard_normal((seq, d_model)).astype(np.float32)

    def body():
        opt.zero_grad()
        out = net(ad.Feeder(lambda: x, shape=[seq, d_model]))
        (out * out * (1.0 / (seq * d_model))).backward()
        opt.step()
    ad.ir_for(range(steps), body)
    res = {}
    Receiver(lambda *a: res.setdefault("params", [v.copy() for v in a]), opt.parameters)
    return res
