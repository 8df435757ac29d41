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


@pytest.mark.parametrize("M,K,N", [(520, 1024, 300), (300, 200, 130), (64, 4096, 64), (5, 70, 33)])
def test_bf16_products_stay_in_bounds(workdir, M, K, N):
    """The bf16 option's operand packs and products (256 x 128 tiles with
    padded operands, K splits, the fp32 tile choice below that)."""
    import numpy as np
    from ad_amd.graph import Receiver, Tensor
    rng = np.random.default_rng(M + K + N)
    a = Tensor(rng.standard_normal((M, K)).astype(np.float32))
    b = Tensor(rng.standard_normal((N, K)).astype(np.float32))
    bias = Tensor(rng.standard_normal((N,)).astype(np.float32))
    Receiver(lambda v: None, [((a @ b.T()) + bias).sigmoid()])
    ok, log = check_run(ad.compile_proc(), workdir, dot_precision="bf16", bf16_min_macs=0)
    assert ok, log


def test_streamed_accesses_stay_in_bounds(workdir):
    """Nontemporal float4 accesses (a reduction and a chain over ranges past
    the streaming threshold, lowered here to 4 KiB)."""
    import numpy as np
    from ad_amd.graph import Receiver, Tensor
    x = Tensor(np.ones((256, 64), np.float32))
    y = Tensor(np.ones((1 << 12,), np.float32))
    Receiver(lambda u, v: None, [x.sum(-1) * 0.5, ((y * 0.5 + 1.0).exp2() + 1.0).recip()])
    ok, log = check_run(ad.compile_proc(), workdir, stream_min_bytes=4096)
    assert ok, log
    assert "ld4<true>" in open([f for f in _sources(workdir)][0]).read()


def _sources(workdir):
    return [os.path.join(workdir, f) for f in os.listdir(workdir) if f.endswith(".cpp")]
