"""Whole training runs of the device computed on the host against the CPU
oracle: every launch, graph replay, staged Feeder input, in-graph copy and
host read of a ``HIPDevice`` run, in the order the device issues them, with
the blocks' threads in lockstep (real barriers, shuffles and fp32 MFMAs;
``host_emulation.LOCKSTEP_SHIM``).  This checks the GPU path's generated
code and its run sequence end to end on the CPU: the MLP of
``examples/linear.py`` (a Feeder in the loop), LayerNorm training (row
reductions) and a batched encoder layer (attention, per-head products,
Feeder input, two steps of one replayed graph)."""
import numpy as np
import pytest

import ad_amd as ad
from ad_amd import workloads
from oracle import OracleDevice

from .host_emulation import host_values


def _host_and_oracle(tmp_path, build, **device_options):
    ad.reset()
    start = build()
    init = [np.array(t.arr, dtype=np.float32).copy() for t in start["params_ref"]] if "params_ref" in start else None
    vals = host_values(ad.compile_proc(), str(tmp_path), lockstep=True, **device_options)
    assert vals is not None, "a launch left the arena or a barrier timed out"
    ad.reset()
    ref = build()
    ad.execute(device=OracleDevice())
    want = [np.asarray(w) for w in ref["params"]]
    # the Receiver of the trained parameters is the run's first host read
    got = [g.reshape(w.shape) for g, w in zip(vals, want)]
    return got, want, init


def _assert_trained_alike(got, want, rtol=1e-4, atol=1e-6):
    for g, w in zip(got, want):
        np.testing.assert_allclose(g, w, rtol=rtol, atol=atol)


def test_mlp_training_steps_on_host(tmp_path):
    """Three SGD steps of Linear-Sigmoid-Linear on a fed [2, 64] input
    (skinny and direct DotProds, the bias-gradient reductions)."""
    build = lambda: workloads.mlp(steps=3, din=64, dh=96, dout=64, rows=2)
    got, want, _ = _host_and_oracle(tmp_path, build)
    assert len(got) == 4
    _assert_trained_alike(got, want)
    # the steps move the weights by far more than the tolerance
    assert max(float(np.max(np.abs(g - w0.reshape(g.shape)))) for g, w0 in zip(got, _initial_mlp())) > 1e-2


def _initial_mlp():
    """The MLP's parameters as ``workloads.mlp`` initialises them."""
    from ad_amd.nn import Linear, Sequential, Sigmoid
    ad.reset()
    params = Sequential(Linear(64, 96), Sigmoid(), Linear(96, 64)).parameters()
    workloads.set_uniform(params, 0)
    return [np.array(p.arr, dtype=np.float32) for p in params]


def test_layernorm_training_steps_on_host(tmp_path):
    """Two steps of LayerNorm training on [64, 256] (row reductions with
    cross-lane sums, their fused epilogues, column sums of the gradients)."""
    build = lambda: workloads.layernorm_train(rows=64, cols=256, steps=2)
    got, want, _ = _host_and_oracle(tmp_path, build)
    assert len(got) == 2
    _assert_trained_alike(got, want)
    gamma, beta = got
    assert np.max(np.abs(gamma - 1.0)) > 1e-2 and np.max(np.abs(beta)) > 1e-2


@pytest.mark.parametrize("options", [
    {},
    {"arena": "unpacked", "graph_dag": True, "stream_min_bytes": 4096},
    {"use_graphs": False, "group_launches": False, "narrow_launches": False},
], ids=["default", "unpacked-dag-streaming", "eager-ungrouped"])
def test_encoder_training_steps_on_host(tmp_path, options):
    """Two steps of a batched encoder layer (2 sequences of 8 rows, d_model
    32, 2 heads, ff 64) with its input fed each step: the per-head and
    attention products, softmax and LayerNorm reductions, the gradient sums
    and the SGD updates -- with the device's defaults, with the unpacked
    arena, dependency-graph replay and nontemporal reads, and launch by
    launch without graphs or grouping.  The learning rate is large so that
    the updates stand far above float32 rounding of the weights."""
    build = lambda: workloads.transformer(layers=1, d_model=32, heads=2, ff=64, seq=8, batch=2,
                                          steps=2, lr=10.0, feeder=True)
    got, want, init = _host_and_oracle(tmp_path, build, **options)
    assert len(got) == len(want) == 15
    for g, w, w0 in zip(got, want, init):
        moved = np.max(np.abs(w - w0.reshape(w.shape)))
        assert moved > 1e-4
        np.testing.assert_allclose(g, w, rtol=0, atol=1e-3 * moved + 1e-7)
