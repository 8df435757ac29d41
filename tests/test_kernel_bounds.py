"""Every kernel launch of whole programs stays inside its allocations, on
the CPU: the device's own plans, arena layout, argument tables and grouped
launches, run on the host under AddressSanitizer (tests/host_emulation.py).
Covers random programs (12 operations, forward and gradients, packed and
unpacked arenas), the transformer, LayerNorm and MLP training loops (graph
replay, Feeder staging, in-loop Receivers), several devices in one process
and a device reused for a second program; a run with the host arena cut
one float short shows the check catches an access past its end."""
import os
import re
import shutil

import pytest

import ad_amd as ad
from ad_amd import workloads

from .fuzz_programs import random_program
from .host_emulation import CLANG, check_run, recording_device

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


@pytest.mark.parametrize("arena", ["packed", "unpacked"])
def test_concat_piece_loads_stay_guarded(workdir, arena):
    """Seed 2008 with gradients: a DotProd epilogue adds a concat whose
    piece reads a slice as ``(g % 100) - 5``; for g % 100 < 5 that index
    underflows, and the piece must only be read where the concat's condition
    selects it.  Its load was hoisted ahead of the condition, an access about
    16 GiB past the buffer (the GPU sweep's illegal memory access)."""
    random_program(2008, n_ops=12, grads=True)
    ok, log = check_run(ad.compile_proc(), workdir, arena=arena)
    assert ok, log


_BUILDERS = {
    "batched": lambda n, r: workloads.transformer(layers=2, d_model=32, heads=4, ff=64, seq=8, batch=2, steps=n,
                                                  receive=r),
    "batched_feeder": lambda n, r: workloads.transformer(layers=1, d_model=32, heads=4, ff=64, seq=8, batch=2,
                                                         steps=n, feeder=True, receive=r),
    "layernorm": lambda n, r: workloads.layernorm_train(rows=64, cols=1024, steps=n, receive=r),
    "mlp": lambda n, r: workloads.mlp(steps=n, receive=r),
}


@pytest.mark.parametrize("build", sorted(_BUILDERS))
def test_training_loops_stay_in_bounds(workdir, build):
    """Whole programs with their ``ir_for`` loops: bodies captured as graphs
    and replayed (an unrolled graph plus single ones, Feeder staging slots
    per iteration), the final Receiver read."""
    _BUILDERS[build](35, True)
    ok, log = check_run(ad.compile_proc(), workdir)
    assert ok, log


def _logged_mlp(steps):
    """A loop body with a Receiver inside (snapshot slots fetched per
    iteration) and a Feeder before it."""
    from ad_amd.graph import Feeder, Receiver
    from ad_amd.nn import Linear, SGD, Sequential, Sigmoid
    import numpy as np
    net = Sequential(Linear(16, 24), Sigmoid(), Linear(24, 8))
    workloads.set_uniform(net.parameters(), 0)
    opt = SGD(net.parameters(), lr=0.01)
    x = np.full((2, 16), 0.2, np.float32)
    seen = []

    def body():
        opt.zero_grad()
        out = net(Feeder(lambda: x, shape=[2, 16]))
        Receiver(lambda v: seen.append(v.copy()), [out.contigious()])
        out.backward()
        opt.step()
    ad.ir_for(range(steps), body)
    return seen


@pytest.mark.parametrize("lag", [0, 1])
def test_loop_with_receiver_stays_in_bounds(workdir, lag):
    seen = _logged_mlp(5)
    ok, log = check_run(ad.compile_proc(), workdir, receiver_lag=lag)
    assert ok, log
    assert len(seen) == 5


def test_several_devices_and_a_reused_one_stay_in_bounds(workdir):
    """Devices made and closed one after another in one process, and one
    device running two programs in turn (its second layout replaces the
    first's arena, tables and graphs)."""
    reused = recording_device()
    for k, seed in enumerate([2000, 2001, 2002]):
        ad.reset()
        random_program(seed, n_ops=12, grads=k % 2 == 1)
        ok, log = check_run(ad.compile_proc(), workdir)
        assert ok, (seed, log)
        ad.reset()
        _BUILDERS["mlp"](3, True) if k % 2 else _BUILDERS["layernorm"](3, True)
        ok, log = check_run(ad.compile_proc(), workdir, device=reused)
        assert ok, (seed, "reused device", log)
    reused.close()


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


@pytest.mark.parametrize("M,K,N,ta,tile", [(640, 1024, 520, False, 128), (300, 2048, 1000, True, 128),
                                           (300, 2048, 64, False, 64), (130, 64, 257, True, 64),
                                           (512, 512, 64, False, 64)])
def test_single_buffer_tiles_stay_in_bounds(workdir, M, K, N, ta, tile):
    """128 x 128 tiles (32-deep panels) and 64 x 64 tiles (64-deep) stage
    their K panels in one LDS buffer (ragged M, N and K, K splits,
    transposed A)."""
    import numpy as np
    from ad_amd.graph import Receiver, Tensor
    rng = np.random.default_rng(M + K + N)
    a = Tensor(rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32))
    b = Tensor(rng.standard_normal((K, N)).astype(np.float32))
    Receiver(lambda v: None, [((a.T() if ta else a) @ b).sigmoid()])
    ok, log = check_run(ad.compile_proc(), workdir, narrow_launches=False)
    assert ok, log
    text = "".join(open(f).read() for f in _sources(workdir))
    assert re.search(rf"dp_mfma<{tile}, {tile}, \d+, {32 if tile == 128 else 64}, LA, LB, EPI, 1>", text)


@pytest.mark.parametrize("M,K,N,ta,tb,copies", [(300, 2048, 64, False, False, 1), (130, 300, 257, True, True, 1),
                                                (512, 512, 64, False, False, 3), (96, 1000, 100, False, True, 1),
                                                (64, 260, 36, True, False, 2),
                                                (512, 64, 512, False, True, 1), (130, 70, 257, True, False, 1)])
def test_narrow_launches_stay_in_bounds(workdir, M, K, N, ta, tb, copies):
    """Launch groups too small to fill the device run ``dp_quad`` (32 x 32
    tiles, 128-deep panels split among the waves): ragged M, N and K, K
    splits, transposed operands, float4 and scalar epilogues, several
    products in one launch."""
    import numpy as np
    from ad_amd.graph import Receiver, Tensor
    rng = np.random.default_rng(M + K + N + copies)
    outs = []
    for _ in range(copies):
        a = Tensor(rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32))
        b = Tensor(rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32))
        bias = Tensor(rng.standard_normal((N,)).astype(np.float32))
        outs.append(((a.T() if ta else a) @ (b.T() if tb else b) + bias).sigmoid())
    Receiver(lambda *v: None, outs)
    ok, log = check_run(ad.compile_proc(), workdir)
    assert ok, log
    text = "".join(open(f).read() for f in _sources(workdir))
    assert re.search(r"dp_quad<\d+, (64|128)>", text) and not re.search(r"dp_mfma<64, 64,", text)


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


def test_wide_streamed_pass_stays_in_bounds(workdir, monkeypatch):
    """A pass of many operands, one element per thread, loading every
    operand nontemporally (thresholds lowered: 2^12 elements, 17 operands)."""
    import numpy as np
    from ad_amd.device.hip import codegen
    from ad_amd.graph import Receiver, Tensor
    monkeypatch.setattr(codegen, "SCALAR_MAX_N", 1024)
    monkeypatch.setattr(codegen, "STREAM_PASS_BYTES", 4096)
    xs = [Tensor(np.full((64, 64), i, np.float32)) for i in range(17)]
    r = xs[0]
    for x in xs[1:]:
        r = r + x
    Receiver(lambda v: None, [r * 0.5])
    ok, log = check_run(ad.compile_proc(), workdir)
    assert ok, log
    text = "".join(open(f).read() for f in _sources(workdir))
    assert text.count("__builtin_nontemporal_load(") >= 17


def _sources(workdir):
    return [os.path.join(workdir, f) for f in os.listdir(workdir) if f.endswith(".cpp")]


@pytest.mark.parametrize("ragged", [False, True])
def test_column_major_gathers_stay_in_bounds(workdir, ragged):
    """Concat operands whose pieces run along the product's rows are
    gathered column-major (threads along the rows, float4 where aligned)."""
    import numpy as np
    from ad_amd.graph import Receiver, Tensor
    rng = np.random.default_rng(11 + ragged)
    M, N = (257, 130) if ragged else (256, 128)
    ka = [61, 67, 128] if ragged else [64, 64, 128]
    A = ad.concat([Tensor(rng.standard_normal((k, M)).astype(np.float32)).T() for k in ka], 1)
    B = ad.concat([Tensor(rng.standard_normal((N, k)).astype(np.float32)).T() for k in ka], 0)
    Receiver(lambda v: None, [(A @ B).sigmoid()])
    ok, log = check_run(ad.compile_proc(), workdir)
    assert ok, log
    text = "".join(open(f).read() for f in _sources(workdir))
    assert text.count("_x = _global_id % ") >= 2
