"""The unpacked arena (``HIPDevice(arena="unpacked")``): every tetris
variable in storage of its own, so launches are ordered by true data flow
only.  Programs are checked against the CPU oracle (which runs the packed
arena) at the parity tolerances, and against the packed HIP run."""
import numpy as np
import pytest

import ad_amd as ad
from ad_amd import workloads
from ad_amd.graph import Receiver, Tensor
from oracle import OracleDevice

from . import programs
from .fuzz_programs import random_program
from .test_fuzz import _close
from .test_hip_parity import assert_params_close

pytestmark = pytest.mark.gpu


def _run(build, device):
    ad.reset()
    out = build()
    ad.execute(device=device)
    return out


BUILDS = {
    "mlp": lambda: programs.mlp(steps=3),
    "layernorm": lambda: programs.layernorm_step(rows=8, cols=16, steps=3),
    "layernorm_wide": lambda: workloads.layernorm_train(rows=64, cols=1024, steps=2),
    "transformer": lambda: programs.transformer(layers=1, d_model=32, heads=4, ff=64, seq=4, steps=2),
    "batched": lambda: workloads.transformer(layers=2, d_model=32, heads=4, ff=64, seq=8, batch=2, steps=3),
}


@pytest.mark.parametrize("name", list(BUILDS))
def test_unpacked_matches_oracle_and_packed(hip, name):
    build = BUILDS[name]
    packed_dev = hip()
    packed = _run(build, packed_dev)
    unpacked_dev = hip(arena="unpacked")
    unpacked = _run(build, unpacked_dev)
    want = _run(build, OracleDevice())
    assert_params_close(unpacked, want)
    assert_params_close(unpacked, packed, rtol=1e-5, atol=1e-6)
    assert unpacked_dev.stats["launches_per_iter"] <= packed_dev.stats["launches_per_iter"]


def test_unpacked_groups_fewer_launches(hip):
    """On a two-layer batched training step the unpacked arena needs fewer
    launches per iteration than the packed one (launches ordered only by
    reuse of memory between variables are merged)."""
    build = BUILDS["batched"]
    packed_dev = hip()
    _run(build, packed_dev)
    unpacked_dev = hip(arena="unpacked")
    _run(build, unpacked_dev)
    assert unpacked_dev.stats["launches_per_iter"] < packed_dev.stats["launches_per_iter"]


@pytest.mark.parametrize("lag", [0, 1])
def test_unpacked_receivers_in_loop(hip, lag):
    a = _run(lambda: programs.mlp_logged(steps=6), hip(arena="unpacked", receiver_lag=lag))
    b = _run(lambda: programs.mlp_logged(steps=6), OracleDevice())
    assert len(a["log"]) == len(b["log"]) == 6
    for x, y in zip(a["log"], b["log"]):
        np.testing.assert_allclose(x, y, rtol=1e-4, atol=1e-5)
    assert_params_close(a, b)


@pytest.mark.parametrize("iters", [7, 50])
def test_unpacked_feeders(hip, iters):
    """Feeder values land in the variable's own storage every iteration
    (unrolled graphs of 32 iterations included).  Exact in fp32."""
    holder = [Tensor(np.zeros((4, 64), dtype=np.float32))]
    count = [0]

    def feed():
        count[0] += 1
        return np.full((4, 64), float(count[0]), dtype=np.float32)

    def body():
        holder[0] += ad.Feeder(feed, shape=[4, 64])
    ad.ir_for(range(iters), body)
    got = {}
    Receiver(lambda v: got.setdefault("acc", v.copy()), [holder[0]])
    ad.execute(device=hip(arena="unpacked"))
    assert count[0] == iters
    assert np.all(got["acc"] == iters * (iters + 1) / 2)


@pytest.mark.parametrize("seed", list(range(0, 30, 3)) + [1000 + s for s in range(0, 20, 2)])
def test_unpacked_random_programs(hip, seed):
    grads = seed >= 1000
    got, _ = _run(lambda: random_program(seed, grads=grads), hip(arena="unpacked"))
    ref, _ = _run(lambda: random_program(seed, grads=grads), OracleDevice())
    assert len(got["outs"]) == len(ref["outs"])
    for x, y in zip(got["outs"], ref["outs"]):
        assert x.shape == y.shape
        _close(x, y)


def test_unpacked_with_bf16_dotprods(hip):
    """Both options together (the fastest configuration bench.py reports):
    a batched transformer trained 3 steps stays within the bf16 tolerance
    of the fp32 oracle (as test_bf16_training_steps)."""
    build = BUILDS["batched"]
    got = _run(build, hip(arena="unpacked", dot_precision="bf16", bf16_min_macs=0))
    want = _run(build, OracleDevice())
    assert_params_close(got, want, rtol=2e-3, atol=2e-3)
