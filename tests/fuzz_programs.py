"""Random programs for parity fuzzing: chains of elementwise, unary,
transpose, slice, concat, reduce and DotProd operations on small random
shapes, traced through the ad front end, with a float64 numpy evaluation of
the same program alongside.

The numpy side follows the reference's semantics where they differ from
plain arithmetic: a reduction combines only the elements its work-group tree
reaches (``tree_inclusion``; all of them for power-of-two lengths) and MAX
pads with 0; ``sqrt`` is ``sqrt(|x|)``; comparisons give 1.0 / 0.0.  Inputs
are in [-1, 1], unary ops are applied where they are well conditioned
(exp2 of a sine, 1 / (x^2 + 1), log2(x^2 + 1)) and products are scaled by
1/sqrt(K), so values stay moderate."""
import numpy as np

import ad_amd as ad
from ad_amd.device.hip.codegen import tree_inclusion
from ad_amd.graph import Receiver, Tensor

DIMS = [1, 2, 3, 4, 5, 8, 12, 16, 17, 32, 64, 100, 130]


def _np_reduce(a, axis, op):
    R = a.shape[axis]
    kept = tree_inclusion(R)
    idx = [y for y in kept if y < R]
    sel = np.take(a, idx, axis=axis)
    if op == "sum":
        return sel.sum(axis=axis)
    out = sel.max(axis=axis)
    if any(y >= R for y in kept):
        out = np.maximum(out, 0.0)
    return out


ALL_KINDS = ("unary", "binary", "scalar", "transpose", "slice", "concat", "reduce", "dot", "broadcast")
# operations whose kernels exchange no data between lanes (no reduction tree,
# no matrix product): their programs compute real values on the host too
LANE_INDEPENDENT_KINDS = ("unary", "binary", "scalar", "transpose", "slice", "concat", "broadcast")


class _Prog:
    def __init__(self, rng, grads, kinds=ALL_KINDS):
        self.rng = rng
        self.grads = grads
        self.kinds = list(kinds)
        self.vals = []          # (node, float64 array)
        self.inputs = []

    def new_input(self, shape):
        arr = self.rng.uniform(-1, 1, shape).astype(np.float32)
        t = Tensor(arr, requires_grad=self.grads)
        self.inputs.append(t)
        self.vals.append((t, arr.astype(np.float64)))
        return self.vals[-1]

    def pick(self, shape=None, ndim=2):
        cands = [v for v in self.vals if len(v[0].shape) == ndim and (shape is None or list(v[0].shape) == list(shape))]
        if cands and self.rng.random() < 0.8:
            return cands[self.rng.integers(len(cands))]
        if shape is None:
            shape = [int(self.rng.choice(DIMS)) for _ in range(ndim)]
        return self.new_input(shape)

    def push(self, node, arr):
        self.vals.append((node, arr))
        return self.vals[-1]

    def step(self):
        rng = self.rng
        kind = rng.choice(self.kinds)
        if kind == "unary":
            x, a = self.pick()
            u = rng.choice(["sin", "exp2", "recip", "log2", "sqrt", "relu", "sigmoid", "gt"])
            if u == "sin":
                return self.push(x.sin(), np.sin(a))
            if u == "exp2":              # exp2 of a value in [-1, 1]
                return self.push(x.sin().exp2(), np.exp2(np.sin(a)))
            if u == "recip":             # 1 / (x^2 + 1)
                return self.push((x * x + 1.0).recip(), 1.0 / (a * a + 1.0))
            if u == "log2":
                return self.push((x * x + 1.0).log2(), np.log2(a * a + 1.0))
            if u == "sqrt":
                return self.push(x.sqrt(), np.sqrt(np.abs(a)))
            if u == "relu":
                return self.push(x.relu(), (a > 0) * a)
            if u == "sigmoid":
                return self.push(x.sigmoid(), 1.0 / (1.0 + np.exp(-a)))
            return self.push(x > 0.25, (a > 0.25).astype(np.float64))
        if kind == "binary":
            x, a = self.pick()
            y, b = self.pick(x.shape)
            if rng.random() < 0.5:
                return self.push(x + y, a + b)
            return self.push(x * y, a * b)
        if kind == "scalar":
            x, a = self.pick()
            c = float(rng.choice([0.5, -1.0, 0.125, 3.0]))
            return self.push(x * c + 0.25, a * c + 0.25)
        if kind == "transpose":
            x, a = self.pick()
            return self.push(x.T(), a.T)
        if kind == "slice":
            x, a = self.pick()
            n = x.shape[0]
            if n < 2:
                return None
            lo = int(rng.integers(0, n - 1))
            hi = int(rng.integers(lo + 1, n + 1))
            return self.push(x[lo:hi], a[lo:hi])
        if kind == "concat":
            x, a = self.pick()
            dim = int(rng.integers(0, 2))
            other = list(x.shape)
            other[dim] = int(rng.choice(DIMS))
            y, b = self.pick(other)
            return self.push(ad.concat([x, y], dim), np.concatenate([a, b], axis=dim))
        if kind == "reduce":
            x, a = self.pick()
            dim = int(rng.integers(0, 2))
            op = "sum" if rng.random() < 0.7 else "max"
            r = x.sum(dim) if op == "sum" else x.max(dim)
            out = _np_reduce(a, dim, op)
            # back to 2-D as a row (dim 1 reduced) or a column
            r2 = r.unsqueeze(dim)
            return self.push(r2 * 0.25, np.expand_dims(out, dim) * 0.25)
        if kind == "dot":
            x, a = self.pick()
            K = x.shape[1]
            N = int(rng.choice(DIMS))
            y, b = self.pick([K, N])
            scale = 1.0 / max(1.0, float(np.sqrt(K)))
            return self.push((x @ y) * scale, (a @ b) * scale)
        if kind == "broadcast":
            x, a = self.pick()
            if x.shape[0] == 1:
                n = int(rng.choice(DIMS))
                return self.push(x.broadcast(0, n), np.broadcast_to(a, (n, a.shape[1])).copy())
            if x.shape[1] == 1:
                n = int(rng.choice(DIMS))
                return self.push(x.broadcast(1, n), np.broadcast_to(a, (a.shape[0], n)).copy())
            return None
        return None


def random_program(seed, n_ops=8, grads=False, kinds=ALL_KINDS):
    """Trace one random program drawing its operations from ``kinds``;
    returns ``(got, expected)``: ``got`` is filled by Receivers when the
    program executes, ``expected`` holds the float64 values of the received
    outputs (None for input gradients, which only a second backend can
    check)."""
    rng = np.random.default_rng(seed)
    p = _Prog(rng, grads, kinds)
    made = []
    while len(made) < n_ops:
        v = p.step()
        if v is not None and len(v[0].shape) == 2:
            made.append(v)
    outs = [v for v in made[-3:]]
    got = {}
    nodes = [v[0].contigious() for v in outs]
    expected = [v[1] for v in outs]
    if grads:
        loss = None
        for v in outs:
            s = (v[0] * v[0]).sum(1).sum(0)
            loss = s if loss is None else loss + s
        loss.backward()
        gnodes = [t.grad() for t in p.inputs if t.grad_tensor is not None]
        nodes += [g.contigious() for g in gnodes]
        expected += [None] * len(gnodes)
    Receiver(lambda *vs: got.setdefault("outs", [x.copy() for x in vs]), nodes)
    return got, expected
