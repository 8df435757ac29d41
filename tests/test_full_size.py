"""Parity at the benchmark configurations' full sizes.

* C1 (examples/linear.py MLP): 1000 SGD steps on the GPU against the CPU
  oracle, parameters within 1e-3 relative.
* C2 single-command benchmarks at their full shapes against float64 numpy
  (sampled rows for the 4096^3 product).
* C3 LayerNorm fwd+bwd [16384,1024] against the oracle, 1 and 100 SGD
  steps (the configuration's own length).
* C4 / C5 transformers at the real shapes: the oracle's naive kernels are
  too slow there, so the steps are restated in float32 torch (the same
  math: per-head projections, per-sample attention scaled by
  1/sqrt(d_model), softmax without max subtraction, post-norm LayerNorm
  with biased variance, ReLU FFN, MSE-to-zero loss, SGD lr 0.01; the
  restatement is checked against the oracle on small stacks below) and
  every updated parameter is compared: after one step (rtol 1e-4 /
  atol 1e-5), after C4's 100 steps and after 10 C5 steps (1e-3 relative).
"""
import numpy as np
import pytest

import ad_amd as ad
from ad_amd import workloads
from oracle import OracleDevice

from . import torch_transformer

gpu = pytest.mark.gpu


def _rel_close(got, want, rel):
    for g, w in zip(got, want):
        scale = max(float(np.abs(w).max()), 1e-30)
        np.testing.assert_allclose(g, w, rtol=0, atol=rel * scale)


@gpu
def test_c1_mlp_1000_steps(hip):
    ad.reset()
    a = workloads.mlp(steps=1000)
    ad.execute(device=hip())
    ad.reset()
    b = workloads.mlp(steps=1000)
    ad.execute(device=OracleDevice())
    assert len(a["params"]) == len(b["params"]) == 4
    _rel_close(a["params"], b["params"], 1e-3)


def _dotprod_bound(a, b, K):
    """Per-element bound on an fp32 sum of K products against float64:
    sqrt(K) * eps * sum_k |a_ik| |b_kj|.  Rounding errors of fp32
    accumulation grow like sqrt(K) for random signs (the worst case K * eps
    is ~60x looser at K = 4096, and admits any sigmoid output); a product
    term dropped or taken with the wrong index moves an element by about
    |a_ik b_kj| ~ 0.64 against a bound of about 0.02 here."""
    return np.sqrt(K) * np.finfo(np.float32).eps * (np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64)))


@gpu
def test_c2_dotprod_elw_full(hip):
    """sigmoid(A@B + bias) on [4096,4096] x [4096,4096]: the pre-activation
    A@B + bias (stored by the same DotProd+Elw command) of 256 sampled rows
    against float64 with a per-element sqrt(K)-scaled bound, and the
    sigmoid of those rows against the float64 sigmoid of the received
    pre-activation (the epilogue alone)."""
    ad.reset()
    out = workloads.dotprod_elw(4096, 4096, 4096, receive_pre=True)
    ad.execute(device=hip())
    a, b, bias = out["inputs"]
    rows = np.random.default_rng(5).choice(4096, 256, replace=False)
    pre = a[rows].astype(np.float64) @ b.astype(np.float64) + bias
    bound = _dotprod_bound(a[rows], b, 4096) + np.finfo(np.float32).eps * np.abs(pre)
    err = np.abs(out["pre"][rows] - pre)
    assert np.all(err <= bound), f"max err/bound {float((err / bound).max()):.3f}"
    assert float(err.max()) > 0.0           # fp32 arithmetic really ran
    got_pre = out["pre"][rows].astype(np.float64)
    want = 1.0 / (1.0 + np.exp2(got_pre * -1.4426950408889634))
    np.testing.assert_allclose(out["r"][rows], want, rtol=2e-6, atol=1e-7)


def test_dotprod_bound_catches_a_dropped_term():
    """The bound of test_c2_dotprod_elw_full rejects a product with one k
    term dropped (planted in a float64 sum on the CPU)."""
    rng = np.random.default_rng(5)
    a = rng.standard_normal((8, 4096), dtype=np.float32)
    b = rng.standard_normal((4096, 64), dtype=np.float32)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    fp32 = (a @ b).astype(np.float64)
    bound = _dotprod_bound(a, b, 4096) + np.finfo(np.float32).eps * np.abs(exact)
    assert np.all(np.abs(fp32 - exact) <= bound)
    dropped = exact - np.outer(a[:, 17], b[17, :])
    assert np.mean(np.abs(dropped - exact) > bound) > 0.9


@gpu
def test_c2_reduce_elw_full(hip):
    ad.reset()
    out = workloads.reduce_elw(8192, 4096, 0.5)
    ad.execute(device=hip())
    (x,) = out["inputs"]
    want = 0.5 * x.astype(np.float64).sum(-1)
    bound = 4096 * np.finfo(np.float32).eps * np.abs(x).sum(-1).max()
    np.testing.assert_allclose(out["r"], want, rtol=0, atol=bound)


@gpu
def test_c2_elw_chain_full(hip):
    ad.reset()
    out = workloads.elw_chain(64 << 20)
    ad.execute(device=hip())
    (x,) = out["inputs"]
    want = 3.0 / (np.exp2(x.astype(np.float64) * 0.5 + 1.0) + 1.0)
    np.testing.assert_allclose(out["r"], want, rtol=2e-6, atol=0)


@gpu
@pytest.mark.parametrize("steps", [1, 100])
def test_c3_layernorm_full(hip, steps):
    """C3 at its own length (100 iterations) and after one: gamma and beta
    against the oracle, rtol 1e-4 / atol 1e-5 after one step, 1e-3
    relative (the bound for long runs) after 100."""
    ad.reset()
    a = workloads.layernorm_train(16384, 1024, steps=steps)
    ad.execute(device=hip())
    ad.reset()
    b = workloads.layernorm_train(16384, 1024, steps=steps)
    ad.execute(device=OracleDevice())
    if steps == 1:
        for x, y in zip(a["params"], b["params"]):
            np.testing.assert_allclose(x, y, rtol=1e-4, atol=1e-5)
    else:
        _rel_close(a["params"], b["params"], 1e-3)


def _reference_steps(res, init, steps, device):
    """The parameters after ``steps`` steps of the float32 torch
    restatement (tests/torch_transformer.py), keyed by parameter id;
    ``device`` "gpu" runs it on the GPU in a child process."""
    order, shape = torch_transformer.flatten(res)
    arrays = [init[id(p)] for p in order]
    if device == "gpu":
        out = torch_transformer.train_on_gpu(arrays, res["x"], shape, steps)
    else:
        out = torch_transformer.train(arrays, res["x"], shape, steps)
    return {id(p): a for p, a in zip(order, out)}


def _torch_step(res, init, lr=0.01):
    """One training step of the traced encoder stack in float32 torch on
    the CPU."""
    return _reference_steps(res, init, 1, "cpu")


@gpu
@pytest.mark.parametrize("config,arena", [("c4", "packed"), ("c5", "packed"), ("c4", "unpacked"),
                                          ("c5", "unpacked")])
def test_transformer_step_full_size_vs_torch(hip, config, arena):
    """One training step at the real shapes: every updated parameter within
    rtol 1e-4 / atol 1e-5 of the float32 torch restatement."""
    layers, d, h, f, s, b = workloads.TRANSFORMER_CONFIGS[config]
    ad.reset()
    res = workloads.transformer(layers=layers, d_model=d, heads=h, ff=f, seq=s, batch=b, steps=1,
                                receive=False)
    init = {id(p): p.arr.copy() for p in res["params_ref"]}
    ad.execute(device=hip(arena=arena))
    want = _reference_steps(res, init, 1, "gpu")
    assert len(want) == len(res["params_ref"])
    for p in res["params_ref"]:
        np.testing.assert_allclose(p.arr, want[id(p)], rtol=1e-4, atol=1e-5)


@gpu
@pytest.mark.parametrize("config,steps", [("c4", 100), ("c5", 10)])
def test_transformer_many_steps_vs_torch(hip, config, steps):
    """C4 at its own length (100 steps in one replayed loop) and C5 for 10:
    every parameter within 1e-3 relative (of its largest magnitude) of the
    float32 torch restatement after the last step."""
    layers, d, h, f, s, b = workloads.TRANSFORMER_CONFIGS[config]
    ad.reset()
    res = workloads.transformer(layers=layers, d_model=d, heads=h, ff=f, seq=s, batch=b, steps=steps,
                                receive=False)
    init = {id(p): p.arr.copy() for p in res["params_ref"]}
    ad.execute(device=hip())
    want = _reference_steps(res, init, steps, "gpu")
    moved = 0.0
    for p in res["params_ref"]:
        w = want[id(p)]
        scale = float(np.abs(w).max())
        np.testing.assert_allclose(p.arr, w, rtol=0, atol=1e-3 * scale)
        moved = max(moved, float(np.abs(w - init[id(p)]).max()) / scale)
    assert moved > 1e-4            # the steps really changed the parameters


@pytest.mark.parametrize("shape", [(2, 32, 4, 64, 8, 2), (1, 16, 2, 32, 4, 4)])
def test_torch_reference_matches_oracle(shape):
    """The torch restatement of the training step used above agrees with the
    CPU oracle on small encoder stacks (so it restates the same graph).
    Every reduction length here is a power of two, as at C4/C5: for other
    lengths the reference's work-group tree drops elements (reduce.py:38-43)
    and a plain sum no longer restates it."""
    layers, d, h, f, s, b = shape
    ad.reset()
    res = workloads.transformer(layers=layers, d_model=d, heads=h, ff=f, seq=s, batch=b, steps=1,
                                receive=False)
    init = {id(p): p.arr.copy() for p in res["params_ref"]}
    ad.execute(device=OracleDevice())
    want = _torch_step(res, init)
    for p in res["params_ref"]:
        np.testing.assert_allclose(p.arr, want[id(p)], rtol=1e-4, atol=1e-6)

