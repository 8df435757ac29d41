"""Values of elementwise passes computed on the host (``host_values``: the
device's own kernels run on the CPU over its arena) against the CPU oracle.

Elementwise kernels exchange no data between lanes, so the host run computes
their real results.  This checks the generated statement code itself on the
CPU -- including heavy passes (more statements than
``codegen.SCALAR_MIN_STMTS`` over at most ``SCALAR_MAX_N`` elements), whose
operand reads are issued in batches ahead of the statements -- before any
GPU run.  Random programs of every kind (DotProds and reductions included)
run with lockstep blocks, which compute cross-lane and MFMA results too."""
import numpy as np
import pytest

import ad_amd as ad
from ad_amd.graph import Receiver, Tensor
from oracle import OracleDevice

from .host_emulation import host_arena, host_values, recording_device


def _chain(seed, n_inputs, n_ops, shape, tweak=None):
    """A chain of elementwise statements over ``n_inputs`` tensors with a
    concat operand, two received intermediate values and the same inputs
    read by many statements; ``tweak`` changes one constant (statement
    ``tweak``)."""
    rng = np.random.default_rng(seed)
    xs = [Tensor(rng.uniform(0.5, 1.5, shape).astype(np.float32)) for _ in range(n_inputs)]
    half = shape[0] // 2
    y = ad.concat([xs[0][:half] * 2.0, xs[1][half:] * 0.5], 0)
    outs = []
    for i in range(n_ops):
        x = xs[int(rng.integers(0, n_inputs))]
        kind = int(rng.integers(0, 5))
        c = 0.75 if i != tweak else 0.7501
        if kind == 0:
            y = y * c + x
        elif kind == 1:
            y = (y * x).sqrt() + 0.25 * c
        elif kind == 2:
            y = y * c + x * xs[i % n_inputs]
        elif kind == 3:
            y = (y * 0.125 * c).exp2() * x
        else:
            y = y * c + (x - 1.0).sin()
        if i in (n_ops // 3, (2 * n_ops) // 3):
            outs.append(y * 1.0)
    outs.append(y)
    got = {}
    Receiver(lambda *v: got.update(v=[a.copy() for a in v]), outs)
    return got


def _host_and_oracle(tmp_path, seed, n_inputs, n_ops, shape, tweak=None):
    ad.reset()
    _chain(seed, n_inputs, n_ops, shape, tweak)
    proc = ad.compile_proc()
    probe = recording_device()
    probe.prepare(proc)
    heavy = sum(p.source.count("__builtin_amdgcn_sched_barrier(0)") for ps in probe.kernels.values() for p in ps)
    ad.reset()
    _chain(seed, n_inputs, n_ops, shape, tweak)
    vals = host_values(ad.compile_proc(), str(tmp_path))
    ad.reset()
    ref = _chain(seed, n_inputs, n_ops, shape)
    ad.execute(device=OracleDevice())
    return heavy, vals, ref["v"]


@pytest.mark.parametrize("seed,n_inputs,n_ops", [(0, 8, 12), (1, 40, 20), (2, 80, 30)])
def test_heavy_pass_values_on_host_match_oracle(tmp_path, seed, n_inputs, n_ops):
    """Heavy passes of one batch and of several (up to 80 inputs plus the
    concat pieces: more reads than one batch of 64)."""
    heavy, vals, ref = _host_and_oracle(tmp_path, seed, n_inputs, n_ops, (128, 128))
    assert heavy >= 1 + (n_inputs > 64), "the program has no (multi-batch) heavy pass"
    assert vals is not None, "a launch left the arena"
    for got, want in zip(vals, ref):
        np.testing.assert_allclose(got.reshape(want.shape), want, rtol=1e-6, atol=1e-6)


def test_host_values_see_a_changed_constant(tmp_path):
    """The check has teeth: the same program with one constant changed
    gives values the oracle's run of the original does not."""
    heavy, vals, ref = _host_and_oracle(tmp_path, 1, 40, 20, (128, 128), tweak=15)
    assert heavy >= 1 and vals is not None
    assert not np.allclose(vals[-1].reshape(ref[-1].shape), ref[-1], rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("transposed,ragged", [(True, False), (True, True), (False, False)])
def test_gathered_concat_operand_on_host(tmp_path, transposed, ragged):
    """The dense copy a large DotProd takes of a concat operand: column-major
    when the pieces run along the product's rows (transposed pieces), else
    row-major; compared element by element with numpy's concatenation."""
    from ad_amd.device.hip import codegen
    ad.reset()
    rng = np.random.default_rng(3 + ragged)
    M, N = (257, 130) if ragged else (256, 128)
    ka = [61, 67, 128] if ragged else [64, 64, 128]
    if transposed:
        pieces = [rng.standard_normal((k, M)).astype(np.float32) for k in ka]
        A = ad.concat([Tensor(x).T() for x in pieces], 1)
        dense = np.concatenate([x.T for x in pieces], 1)
    else:
        pieces = [rng.standard_normal((M, k)).astype(np.float32) for k in ka]
        A = ad.concat([Tensor(x) for x in pieces], 1)
        dense = np.concatenate(pieces, 1)
    B = Tensor(rng.standard_normal((sum(ka), N)).astype(np.float32))
    Receiver(lambda v: None, [A @ B])
    assert M * N * sum(ka) >= codegen.GATHER_MIN_MACS
    dev, arena = host_arena(ad.compile_proc(), str(tmp_path))
    assert arena is not None, "a launch left the arena"
    (pid, plans), = [(pid, ps) for pid, ps in dev.kernels.items()
                     if any(p.family == "dotprod" for p in ps) and ps[0].family == "elw"]
    gather = plans[0]
    col_major = "_x = _global_id % " in gather.source
    assert col_major == transposed
    dst = next(i for i, a in enumerate(gather.args) if a[0] == "scratch")
    off = dev._arg_values(gather, pid)[dst][1]
    got = arena[off:off + 4 * dense.size].view(np.float32)
    want = dense.T.ravel() if col_major else dense.ravel()
    assert np.array_equal(got, want)


@pytest.mark.parametrize("seed", range(24))
def test_random_lane_independent_programs_on_host(tmp_path, seed):
    """Random chains of unary, binary, scalar, transpose, slice, concat and
    broadcast operations (the fuzz generator restricted to lane-independent
    kinds; float4 and scalar passes, concat conditions, permuted and sliced
    reads): every received value of the host run equals the oracle's."""
    from .fuzz_programs import LANE_INDEPENDENT_KINDS, random_program
    ad.reset()
    random_program(3000 + seed, n_ops=14, kinds=LANE_INDEPENDENT_KINDS)
    vals = host_values(ad.compile_proc(), str(tmp_path))
    assert vals is not None, "a launch left the arena"
    ad.reset()
    ref, _ = random_program(3000 + seed, n_ops=14, kinds=LANE_INDEPENDENT_KINDS)
    ad.execute(device=OracleDevice())
    assert len(vals) >= len(ref["outs"])
    for got, want in zip(vals, ref["outs"]):
        np.testing.assert_allclose(got.reshape(want.shape), want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("seed", [0, 3, 7, 12, 17, 25, 1001, 1006, 1011, 1016])
def test_random_programs_in_lockstep_on_host(tmp_path, seed):
    """Random programs of every kind the generator has (DotProds and
    reductions included; gradients from seed 1000 on, as in the GPU fuzz
    test), run on the host with lockstep blocks: every received value
    equals the oracle's to the GPU test's tolerance."""
    from .fuzz_programs import random_program
    grads = seed >= 1000
    ad.reset()
    random_program(seed, grads=grads)
    vals = host_values(ad.compile_proc(), str(tmp_path), lockstep=True)
    assert vals is not None, "a launch left the arena or a barrier timed out"
    ad.reset()
    ref, _ = random_program(seed, grads=grads)
    ad.execute(device=OracleDevice())
    assert len(vals) >= len(ref["outs"])
    for got, want in zip(vals, ref["outs"]):
        scale = max(1.0, float(np.abs(want).max()) if want.size else 1.0)
        np.testing.assert_allclose(got.reshape(want.shape), want, rtol=1e-4, atol=1e-4 * scale)
