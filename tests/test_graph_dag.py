"""Loop bodies replayed as dependency graphs (``HIPDevice(graph_dag=True)``):
on the CPU, against a recording context, every pair of captured nodes that
touch overlapping memory -- one of them writing -- must stay ordered in the
graph (one reaches the other along the dependency edges), and every copy
(a Feeder's staging slot, a Receiver's snapshot) is ordered against every
other node.  Covers unrolled bodies (several iterations per graph), bodies
with Feeders and Receivers, and the transformer step."""
import pytest

import ad_amd as ad
from ad_amd import workloads
from ad_amd.graph import Feeder, ForNode, Receiver

from .host_emulation import recording_device
from .test_kernel_bounds import _logged_mlp


def _overlap(a, b):
    return any(x[0] == y[0] and x[1] < y[2] and y[1] < x[2] for x in a for y in b)


def _conflict(u, v):
    (ur, uw), (vr, vw) = u, v
    return _overlap(uw, vw) or _overlap(uw, vr) or _overlap(ur, vw)


def _nodes(dev, inner, count):
    """Per captured node, in capture order: ("launch", reads, writes) or
    ("copy",), walking the schedule as the capture does."""
    out = []
    stretches = dev.stretch_graphs.get(inner.id, [])
    s = -1
    for _ in range(count):
        s = -1
        for item in dev._schedules[inner.id]:
            if item[0] == "launch":
                g, makes_node = item[3], item[5]
                if g == 0:
                    s += 1
                if makes_node:
                    _, _, _, reads, writes, _ = stretches[s][g]
                    out.append(("launch", reads, writes))
            elif isinstance(item[1], Receiver):
                out.extend(("copy",) for _ in item[1].ids)
            elif isinstance(item[1], Feeder):
                out.append(("copy",))
    return out


def _check(dev, proc):
    ctx = dev.ctx
    assert not ctx.errors, ctx.errors
    loop = [c for c in proc.procedure if isinstance(c, ForNode)][0]
    inner = loop.get_proc()
    dags = ctx.dags
    assert dags, "no graph was captured"
    checked = 0
    for deps in dags:
        count = 1
        per_iter = len(_nodes(dev, inner, 1))
        if per_iter and len(deps) != per_iter:
            count = len(deps) // per_iter
        nodes = _nodes(dev, inner, count)
        assert len(nodes) == len(deps)
        reach = []                       # reach[i]: bit j set when node j precedes node i
        for i, d in enumerate(deps):
            bits = 0
            for j in d:
                bits |= reach[j] | (1 << j)
            reach.append(bits)
        for i in range(len(nodes)):
            for j in range(i):
                if nodes[i][0] == "copy" or nodes[j][0] == "copy" or \
                        _conflict(nodes[j][1:], nodes[i][1:]):
                    assert reach[i] >> j & 1, f"nodes {j} and {i} touch the same memory but are not ordered"
                    checked += 1
    return checked


@pytest.mark.parametrize("build", ["transformer", "layernorm", "mlp_unrolled", "logged_mlp", "feeder_transformer"])
def test_graph_orders_every_conflict(build):
    builders = {
        "transformer": lambda: workloads.transformer(layers=2, d_model=32, heads=4, ff=64, seq=8, batch=2, steps=3),
        "layernorm": lambda: workloads.layernorm_train(rows=64, cols=256, steps=3),
        "mlp_unrolled": lambda: workloads.mlp(steps=40, din=16, dh=24, dout=8),
        "logged_mlp": lambda: _logged_mlp(4),
        "feeder_transformer": lambda: workloads.transformer(layers=1, d_model=32, heads=4, ff=64, seq=8, batch=2,
                                                            steps=3, feeder=True),
    }
    builders[build]()
    proc = ad.compile_proc()
    dev = recording_device(graph_dag=True)
    dev.execute(proc)
    assert _check(dev, proc) > 0


def test_graph_is_sparser_than_the_chain():
    """The transformer step's graph lets launches run side by side: fewer
    edges on its longest path than nodes."""
    workloads.transformer(layers=2, d_model=32, heads=4, ff=64, seq=8, batch=2, steps=2, receive=False)
    proc = ad.compile_proc()
    dev = recording_device(graph_dag=True)
    dev.execute(proc)
    deps = dev.ctx.dags[0]
    depth = []
    for d in deps:
        depth.append(1 + max((depth[j] for j in d), default=0))
    assert max(depth) < len(deps)


@pytest.mark.gpu
@pytest.mark.parametrize("build", ["transformer", "logged_mlp"])
def test_dag_graph_matches_the_oracle(hip, build):
    """The dependency-graph replay gives the oracle's results (a training
    loop; a body with a Feeder and an in-loop Receiver)."""
    import numpy as np
    from oracle import OracleDevice
    if build == "transformer":
        def make():
            return workloads.transformer(layers=2, d_model=32, heads=4, ff=64, seq=8, batch=2, steps=4)
    else:
        def make():
            return {"seen": _logged_mlp(6)}
    ad.reset()
    got = make()
    ad.execute(device=hip(graph_dag=True))
    ad.reset()
    ref = make()
    ad.execute(device=OracleDevice())
    key = "params" if build == "transformer" else "seen"
    assert len(got[key]) == len(ref[key]) > 0
    for x, y in zip(got[key], ref[key]):
        np.testing.assert_allclose(x, y, rtol=1e-4, atol=1e-5)
