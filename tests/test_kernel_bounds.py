"""Every kernel launch of whole programs stays inside its allocations, on
the CPU: the device's own plans, arena layout, argument tables and grouped
launches, run on the host under AddressSanitizer (tests/host_emulation.py).
Covers random programs (12 operations, forward and gradients, packed and
unpacked arenas) and the transformer, LayerNorm and MLP steps; a run with
the host arena cut one float short shows the check catches an access past
its end."""
import os
import shutil

import pytest

import ad_amd as ad
from ad_amd import workloads

from .fuzz_programs import random_program
from .host_emulation import CLANG, check_run

pytestmark = pytest.mark.skipif(not os.path.exists(CLANG), reason="needs the ROCm host clang")


@pytest.fixture
def workdir(tmp_path):
    yield str(tmp_path)
    shutil.rmtree(tmp_path, ignore_errors=True)


@pytest.mark.parametrize("seed", [2000, 2001, 2002, 2003, 2004, 2005])
@pytest.mark.parametrize("arena", ["packed", "unpacked"])
def test_random_programs_stay_in_bounds(workdir, seed, arena):
    random_program(seed, n_ops=12, grads=seed % 2 == 1)
    ok, log = check_run(ad.compile_proc(), workdir, arena=arena)
    assert ok, log


@pytest.mark.parametrize("build", ["batched", "layernorm", "mlp"])
def test_training_steps_stay_in_bounds(workdir, build):
    builders = {
        "batched": lambda: workloads.transformer(layers=2, d_model=32, heads=4, ff=64, seq=8, batch=2, steps=1,
                                                 receive=False),
        "layernorm": lambda: workloads.layernorm_train(rows=64, cols=1024, steps=1, receive=False),
        "mlp": lambda: workloads.mlp(steps=1, receive=False),
    }
    builders[build]()
    proc = ad.compile_proc()
    # the loop body runs once: the emulation replays no graphs
    from ad_amd.graph import ForNode
    body = []
    for c in proc.procedure:
        body.extend(c.get_proc().procedure if isinstance(c, ForNode) else [c])
    proc.procedure = body
    ok, log = check_run(proc, workdir)
    assert ok, log


def test_an_access_past_the_arena_is_caught(workdir):
    random_program(2002, n_ops=12)
    ok, log = check_run(ad.compile_proc(), workdir, shrink=4)
    assert not ok and "AddressSanitizer" in log
