"""The CPU oracle against the reference's known answers and against closed
forms in float64 numpy.  These pin the oracle before it is used to judge
the HIP backend."""
import math
import pathlib

import numpy as np
import pytest

import ad_amd as ad
from ad_amd.graph import Receiver, Tensor
from ad_amd.nn import LayerNorm
from oracle import OracleDevice

from . import programs

GOLDEN = pathlib.Path(__file__).parent / "golden"


def run():
    ad.execute(device=OracleDevice())


def test_known_answer_dotprod():
    """reference tests/dotprod_test.py:8-9"""
    d = np.load(GOLDEN / "dotprod_test_inputs.npz")
    inp = Tensor(d["inp"], requires_grad=True)
    w = Tensor(d["weight"], requires_grad=True)
    b = Tensor(d["bias"], requires_grad=True)
    r = (inp @ w) + b
    r.backward()
    got = {}
    Receiver(lambda res, g: got.update(r=res.copy(), g=g.copy()), [r, inp.grad()])
    run()
    assert round(float(got["r"].sum()), 4) == -3.2747
    assert round(float(got["g"].sum()), 4) == 8.2885


def _temp_through_permute_program():
    """``(x*2).T() * y`` in one ElwFuse with y = 1: the product's left
    operand is the fused temp ``x*2`` read through a transpose."""
    x = Tensor(np.arange(16, dtype=np.float32).reshape(4, 4))
    y = Tensor(np.ones((4, 4), dtype=np.float32))
    got = {}
    Receiver(lambda v: got.setdefault("v", v.copy()), [((x * 2.0).T() * y).contigious()])
    return got


TEMP_QUIRK_ANSWER = 2.0 * np.arange(16, dtype=np.float32).reshape(4, 4)


def test_known_answer_temp_read_through_permute():
    """The reference lowers a fused temp as ``temp_<id>`` whatever its
    access (karg.py:47-48), so the transposed read of ``x*2`` inside the
    fusion yields each element's own ``2*x[i][j]``: by hand, row i is
    2*(4i, 4i+1, 4i+2, 4i+3), not the transpose 2*(i, i+4, i+8, i+12)."""
    got = _temp_through_permute_program()
    run()
    assert np.array_equal(got["v"], TEMP_QUIRK_ANSWER)
    assert not np.array_equal(got["v"], TEMP_QUIRK_ANSWER.T)


def test_known_answer_unary():
    """reference tests/unary_test.py:11-14"""
    inp = Tensor(np.array([[0.3, 0.2, 0.7, 0.54], [0.13, 0.77, 0.23, 0.22]]), requires_grad=True)
    result = inp.exp2() + 3
    result = result.sqrt().recip() * -2.5 + result.log2()
    result = result.sin()
    result_two = (inp > 0.5) * inp.exp2()
    result.backward()
    result_two.backward()
    got = {}
    Receiver(lambda a, b, c: got.update(a=a.copy(), b=b.copy(), c=c.copy()), [result, result_two, inp.grad()])
    run()
    assert round(float(got["a"].sum()), 5) == 6.2689
    assert round(float(got["b"].sum()), 5) == 4.78375
    assert round(float(got["c"].sum()), 5) == 5.39896


def test_known_answer_layernorm():
    """reference tests/layernorm_test.py:19-22"""
    x = Tensor(np.array([[5.0, 6.0, 3.0], [4.0, 5.0, 6.0]]), requires_grad=True)
    ln = LayerNorm(3)
    res = ln(x)
    res.backward()
    got = {}
    Receiver(lambda a, b, c: got.update(y=a.copy(), db=b.copy(), ds=c.copy()),
             [res, ln.bias.grad().contigious(), ln.scale.grad().contigious()])
    run()
    assert round(float(got["y"].flatten()[0]), 4) == 0.2673
    assert round(float(got["db"].flatten()[0]), 4) == 2.0
    assert round(float(got["ds"].flatten()[0]), 4) == -0.9575


def test_known_answer_pow2_and_concat():
    """reference tests/powtwo_test.py:18-27, variance_test.py:19-28,
    concat_test.py:28-34 (exact)."""
    x = Tensor(np.array([[5.0, 6.0, 3.0], [4.0, 5.0, 6.0]]), requires_grad=True)
    res = x.pow2()
    res.backward()
    got = {}
    Receiver(lambda r, g: got.update(r=r.copy(), g=g.copy()), [res, x.grad()])
    run()
    assert np.array_equal(got["r"], [[25, 36, 9], [16, 25, 36]])
    assert np.array_equal(got["g"], [[10, 12, 6], [8, 10, 12]])
    ad.reset()
    x = Tensor(np.array([[5.0, 6.0, 3.0, 1.0], [4.0, 5.0, 6.0, 3.0]]), requires_grad=True)
    y = Tensor(np.array([[8.0, 9.0, 3.0, 6.0], [3.0, 5.0, 4.0, 2.0]]), requires_grad=True)
    res = ad.concat([x * 2, y * 3], 1).contigious()
    res.backward()
    Receiver(lambda r, xg, yg: got.update(c=r.copy(), xg=xg.copy(), yg=yg.copy()), [res, x.grad(), y.grad()])
    run()
    assert np.array_equal(got["c"], [[10, 12, 6, 2, 24, 27, 9, 18], [8, 10, 12, 6, 9, 15, 12, 6]])
    assert got["xg"].sum() == 16 and got["yg"].sum() == 24


def _np_mlp(params, steps, x, lr=0.01):
    """examples/linear.py in float64: loss = sum(out), SGD."""
    w1, b1, w2, b2 = [p.astype(np.float64) for p in params]
    for _ in range(steps):
        h = x @ w1 + b1
        s = 1.0 / (1.0 + np.exp(-h))
        g_out = np.ones((x.shape[0], w2.shape[1]))
        gw2 = s.T @ g_out
        gb2 = g_out.sum(0)
        gs = g_out @ w2.T
        gh = gs * s * (1 - s)
        gw1 = x.T @ gh
        gb1 = gh.sum(0)
        w1, b1, w2, b2 = w1 - lr * gw1, b1 - lr * gb1, w2 - lr * gw2, b2 - lr * gb2
    return w1, b1, w2, b2


def test_mlp_closed_form():
    """Config 1 (examples/linear.py) for 5 steps vs float64 numpy.  The
    parameter order in the Receiver is Module.parameters() order."""
    out = programs.mlp(steps=5)
    # the same initial weights, regenerated
    ad.reset()
    from ad_amd.nn import Linear, Sequential, Sigmoid
    net = Sequential(Linear(255, 255), Sigmoid(), Linear(255, 255))
    programs.set_uniform(net.parameters(), 0)
    l1, l2 = net.modules[0], net.modules[2]
    init = [l1.w.arr.copy(), l1.b.arr.copy(), l2.w.arr.copy(), l2.b.arr.copy()]
    ad.reset()
    out = programs.mlp(steps=5)
    run()
    x = np.full((2, 255), 0.2)
    ref = _np_mlp(init, 5, x)
    for got, want in zip(out["params"], ref):
        np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-6)


def test_layernorm_closed_form():
    """LN forward and gamma/beta gradients vs float64 numpy."""
    rng = np.random.default_rng(1)
    xv = rng.standard_normal((16, 32)).astype(np.float32)
    dyv = rng.standard_normal((16, 32)).astype(np.float32)
    x = Tensor(xv)
    dy = Tensor(dyv)
    ln = LayerNorm(32)
    y = ln(x)
    (y * dy).backward()
    got = {}
    Receiver(lambda a, b, c: got.update(y=a.copy(), db=b.copy(), ds=c.copy()),
             [y, ln.bias.grad().contigious(), ln.scale.grad().contigious()])
    run()
    x64 = xv.astype(np.float64)
    mu = x64.mean(1, keepdims=True)
    var = ((x64 - mu) ** 2).mean(1, keepdims=True)
    xn = (x64 - mu) / np.sqrt(var + 1e-5)
    np.testing.assert_allclose(got["y"], xn, rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(got["db"], dyv.sum(0), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(got["ds"], (dyv * xn).sum(0), rtol=1e-4, atol=1e-4)


def test_softmax_attention_closed_form():
    """One attention head: softmax(Q K^T / sqrt(d)) V (no max subtraction,
    scale 1/sqrt(d_model)) vs float64 numpy.  Eight keys: the reference's
    row sum is exact only for power-of-two work-groups (A.1)."""
    from ad_amd.nn import Attention
    rng = np.random.default_rng(3)
    q, k, v = (rng.standard_normal((8, 8)).astype(np.float32) for _ in range(3))
    out = Attention()(Tensor(q), Tensor(k), Tensor(v), 32)
    got = {}
    Receiver(lambda o: got.setdefault("o", o.copy()), [out])
    run()
    s = q.astype(np.float64) @ k.T.astype(np.float64) / math.sqrt(32.0)
    p = np.exp(s) / np.exp(s).sum(1, keepdims=True)
    np.testing.assert_allclose(got["o"], p @ v, rtol=1e-5, atol=1e-5)


def test_reduce_tree_drops_like_reference():
    """reduce.py:38-43 with R=5: L=6, the tree drops element 2 (A.1); R=3
    and R=4 sum everything."""
    for r, dropped in ((5, [2]), (3, []), (4, []), (6, [2, 5][:0])):
        ad.reset()
        xv = np.arange(1, 2 * r + 1, dtype=np.float32).reshape(2, r)
        s = Tensor(xv).sum(-1)
        got = {}
        Receiver(lambda a: got.setdefault("s", a.copy()), [s])
        run()
        keep = [i for i in range(r) if i not in dropped]
        if r == 6:
            keep = [0, 1, 3, 4]     # L=6: slots 2 and 5 never reach slot 0
        np.testing.assert_array_equal(got["s"], xv[:, keep].sum(1))


def test_lockstep_equals_workitem_when_no_hazard():
    """The timed work-item form of each kernel equals the lockstep form on a
    program without in-kernel aliasing (the MLP)."""
    out_a = programs.mlp(steps=2)
    ad.execute(device=OracleDevice(lockstep=True))
    ad.reset()
    out_b = programs.mlp(steps=2)
    ad.execute(device=OracleDevice(lockstep=False))
    for a, b in zip(out_a["params"], out_b["params"]):
        np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("R", [5, 6, 1000, 1024])
def test_exact_reduce_mode_sums_every_element(R):
    """With exact_reduce the oracle combines all R elements: SUM matches a
    float64 sum and MAX over all-negative rows is the true maximum (the
    reference's tree drops elements for R = 5, 6, 1000 and pads MAX with 0)."""
    import ad_amd as ad
    from ad_amd.graph import Receiver, Tensor
    from oracle import OracleDevice
    ad.reset()
    rng = np.random.default_rng(R)
    a = rng.standard_normal((7, R)).astype(np.float32)
    neg = -np.abs(a) - 0.5
    got = {}
    Receiver(lambda s, m: got.update(s=s.copy(), m=m.copy()),
             [Tensor(a).sum(-1), Tensor(neg).max(-1)])
    ad.execute(device=OracleDevice(exact_reduce=True))
    np.testing.assert_allclose(got["s"], a.astype(np.float64).sum(-1), rtol=1e-5, atol=1e-4)
    assert np.array_equal(got["m"], neg.max(-1))
    ad.reset()
