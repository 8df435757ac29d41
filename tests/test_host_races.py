"""Data shared between the threads of a block is ordered by barriers, and
the blocks of a launch do not depend on each other: the generated kernels
run on the host in lockstep twice, with a launch's blocks run and a block's
threads resumed in ascending and in descending order (``host_emulation``
with ``descending``), and every host read is bit-identical.  A write to LDS
read by another thread without a barrier in between gives different results
in the two orders, as do lanes of one wave that exchange data without a
wavefront fence, and blocks (or grouped instances of one launch) that read
what another block of the launch writes.  Runs on several streams are also
replayed with the later streams' work moved as early as their event waits
allow, and loop bodies replayed as dependency graphs with the latest ready
node run first."""
import numpy as np
import pytest

import ad_amd as ad
from ad_amd import workloads
from ad_amd.graph import Receiver, Tensor

from .host_emulation import host_values


def _product(M, K, N, ta, tb):
    """A product with a fused epilogue and both reductions of it."""
    rng = np.random.default_rng(M + K + N)
    a = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    b = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    A, B = Tensor(a), Tensor(b)
    r = (A.T() if ta else A) @ (B.T() if tb else B)
    Receiver(lambda *v: None, [(r + 1.0).sigmoid(), r.sum(0), r.sum(1)])


CASES = {
    "layernorm-training": (lambda: workloads.layernorm_train(rows=64, cols=256, steps=2), {}, "reduce_rows<"),
    # grouped launches, and the loop body replayed as a dependency graph
    "encoder-training-dag": (lambda: workloads.transformer(layers=1, d_model=32, heads=2, ff=64, seq=8, batch=2,
                                                           steps=2, lr=10.0, feeder=True), {"graph_dag": True},
                             "reduce_cols<"),
    "tile64": (lambda: _product(130, 300, 257, True, False), {"narrow_launches": False}, "dp_mfma<64, 64"),
    "tile128": (lambda: _product(520, 136, 520, True, True), {"narrow_launches": False}, "dp_mfma<128, 128"),
    "quad": (lambda: _product(130, 300, 257, True, True), {}, "dp_quad<1, 128>"),
    "quad-split": (lambda: _product(64, 1024, 64, False, True), {}, "dp_quad<4, 128>"),
    "bf16": (lambda: _product(130, 70, 257, True, True), {"dot_precision": "bf16", "bf16_min_macs": 0}, "dp_bf16<"),
}


@pytest.mark.parametrize("name", list(CASES))
def test_thread_order_does_not_change_results(tmp_path, name):
    build, options, kernel = CASES[name]
    runs = []
    for descending in (False, True):
        ad.reset()
        build()
        proc = ad.compile_proc()
        workdir = tmp_path / ("descending" if descending else "ascending")
        workdir.mkdir()
        runs.append(host_values(proc, str(workdir), lockstep=True, descending=descending, **options))
        assert runs[-1] is not None, "a launch left the arena or a barrier no thread could pass"
    sources = " ".join(open(p).read() for p in tmp_path.glob("ascending/run_*.cpp"))
    assert kernel in sources
    up, down = runs
    assert len(up) == len(down) > 0
    for x, y in zip(up, down):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))


def test_stream_waits_order_the_lanes(tmp_path):
    """Uncaptured runs on several streams (``lanes=4``, no graphs): two
    training steps of an encoder layer run in the order the device
    issues them and again with the operations of the later streams run as
    early as their event waits allow (``lanes_late_first``), blocks and
    threads in descending order.  Both agree bit for bit, and with the
    oracle: the waits the scheduler places order every dependent launch."""
    from oracle import OracleDevice
    from .host_emulation import recording_device
    build = lambda: workloads.transformer(layers=1, d_model=32, heads=2, ff=64, seq=8, batch=2, steps=2,
                                          lr=10.0, feeder=True)
    options = {"lanes": 4, "use_graphs": False}
    ad.reset()
    build()
    probe = recording_device(**options)
    probe.execute(ad.compile_proc())
    assert probe.stats["lanes_used"] >= 3
    assert sum(op[0] == "wait" for op in probe.ctx.launches) > 0
    runs = []
    for descending in (False, True):
        ad.reset()
        build()
        workdir = tmp_path / ("late-first" if descending else "issued")
        workdir.mkdir()
        runs.append(host_values(ad.compile_proc(), str(workdir), lockstep=True, descending=descending, **options))
        assert runs[-1] is not None, "a launch left the arena or a barrier no thread could pass"
    for x, y in zip(*runs):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
    ad.reset()
    ref = build()
    ad.execute(device=OracleDevice())
    for got, want in zip(runs[1], ref["params"]):
        np.testing.assert_allclose(got.reshape(np.shape(want)), want, rtol=1e-5, atol=1e-6)
