"""Parity of the HIP backend with the CPU oracle on identical programs.

Tolerances: data movement and +,* chains are bit-exact; anything through a
dot product or reduction (reassociated on the GPU) or a libm function
(exp2/log2/sin differ by ulps between glibc and the ROCm device library) is
checked at rtol 1e-4 / atol 1e-5 per step."""
import pathlib

import numpy as np
import pytest

import ad_amd as ad
from ad_amd.graph import Receiver, Tensor
from oracle import OracleDevice

from . import programs

GOLDEN = pathlib.Path(__file__).parent / "golden"

pytestmark = pytest.mark.gpu


def run_both(build, hip):
    ad.reset()
    out_hip = build()
    ad.execute(device=hip())
    ad.reset()
    out_cpu = build()
    ad.execute(device=OracleDevice())
    return out_hip, out_cpu


def assert_params_close(a, b, rtol=1e-4, atol=1e-5):
    assert len(a["params"]) == len(b["params"])
    for x, y in zip(a["params"], b["params"]):
        np.testing.assert_allclose(x, y, rtol=rtol, atol=atol)


@pytest.mark.parametrize("M,K,N", [(2, 255, 255), (128, 64, 128), (130, 70, 257), (256, 512, 64), (1, 3, 1),
                                   (8, 1000, 300), (5, 17, 64), (9, 40, 33), (300, 2, 200), (64, 8, 130)])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_dotprod_shapes(hip, M, K, N, ta, tb):
    """A @ B through the MFMA template (and, for at most 8 rows or at most 8
    terms, the skinny and direct ones) for row-major and transposed
    operands, against float64 numpy with a K-scaled bound."""
    rng = np.random.default_rng(M * 7 + K * 3 + N)
    a = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    b = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    A = Tensor(a)
    B = Tensor(b)
    r = (A.T() if ta else A) @ (B.T() if tb else B)
    got = {}
    Receiver(lambda v: got.setdefault("r", v.copy()), [r])
    ad.execute(device=hip())
    ref = (a.T if ta else a).astype(np.float64) @ (b.T if tb else b).astype(np.float64)
    bound = 4 * K * np.finfo(np.float32).eps * (np.abs(a).max() * np.abs(b).max()) + 1e-6
    np.testing.assert_allclose(got["r"], ref, rtol=0, atol=bound)


@pytest.mark.parametrize("M,K,N,ta,tb,copies", [(300, 2048, 64, False, False, 1), (130, 300, 257, True, True, 1),
                                                (512, 512, 64, False, False, 3), (96, 1000, 100, False, True, 1),
                                                (64, 260, 36, True, False, 2),
                                                (512, 64, 512, False, True, 1), (130, 70, 257, True, False, 1), (512, 512, 64, True, True, 16)])
def test_narrow_launch_parity(hip, M, K, N, ta, tb, copies):
    """Launch groups too small to fill the device run ``dp_quad`` (32 x 32
    tiles, each block's K panels split among its four waves, partial tiles
    added through LDS): the pre-activation ``A@B + bias`` of every product
    against float64 within sqrt(K)·eps·Σ_k|a||b| per element, the sigmoid
    epilogue against the float64 sigmoid of the received pre-activation,
    and the whole output against the 64 x 64-tile kernel's (narrow
    launches off) within fp32 rounding of a regrouped sum."""
    rng = np.random.default_rng(M + K + N + copies)
    data = []
    for _ in range(copies):
        a = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
        b = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
        data.append((a, b, rng.standard_normal((N,)).astype(np.float32)))

    def build():
        outs, got = [], {}
        for a, b, bias in data:
            A, B, C = Tensor(a), Tensor(b), Tensor(bias)
            pre = (A.T() if ta else A) @ (B.T() if tb else B) + C
            outs += [pre, pre.sigmoid()]
        Receiver(lambda *v: got.setdefault("v", [x.copy() for x in v]), outs)
        return got

    runs = {}
    for narrow in (True, False):
        ad.reset()
        got = build()
        dev = hip(narrow_launches=narrow)
        ad.execute(device=dev)
        names = " ".join(p.source for p in dev._narrow_plans.values())
        assert ("dp_quad" in names) == narrow
        runs[narrow] = got["v"]
    eps = np.finfo(np.float32).eps
    for i, (a, b, bias) in enumerate(data):
        a64 = (a.T if ta else a).astype(np.float64)
        b64 = (b.T if tb else b).astype(np.float64)
        ref = a64 @ b64 + bias
        bound = np.sqrt(K) * eps * (np.abs(a64) @ np.abs(b64)) + 4 * eps * np.abs(bias)
        pre, sig = runs[True][2 * i], runs[True][2 * i + 1]
        assert np.all(np.abs(pre - ref) <= bound), f"product {i}: {np.max(np.abs(pre - ref) / bound):.3f} x bound"
        np.testing.assert_allclose(sig, 1 / (1 + np.exp(-pre.astype(np.float64))), rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(pre, runs[False][2 * i], rtol=0, atol=float(np.max(bound)))


def test_reference_known_answers_dotprod(hip):
    """tests/dotprod_test.py:8-9 of the reference (torch seed 42 inputs)."""
    d = np.load(GOLDEN / "dotprod_test_inputs.npz")
    inp = Tensor(d["inp"], requires_grad=True)
    w = Tensor(d["weight"], requires_grad=True)
    b = Tensor(d["bias"], requires_grad=True)
    r = (inp @ w) + b
    r.backward()
    got = {}
    Receiver(lambda res, g: got.update(r=res.copy(), g=g.copy()), [r, inp.grad()])
    ad.execute(device=hip())
    assert round(float(got["r"].sum()), 4) == -3.2747
    assert round(float(got["g"].sum()), 4) == 8.2885


def test_reference_known_answers_unary(hip):
    """tests/unary_test.py:11-14 of the reference."""
    inp = Tensor(np.array([[0.3, 0.2, 0.7, 0.54], [0.13, 0.77, 0.23, 0.22]]), requires_grad=True)
    result = inp.exp2() + 3
    result = result.sqrt().recip() * -2.5 + result.log2()
    result = result.sin()
    result_two = (inp > 0.5) * inp.exp2()
    result.backward()
    result_two.backward()
    got = {}
    Receiver(lambda a, b, c: got.update(a=a.copy(), b=b.copy(), c=c.copy()), [result, result_two, inp.grad()])
    ad.execute(device=hip())
    assert round(float(got["a"].sum()), 5) == 6.2689
    assert round(float(got["b"].sum()), 5) == 4.78375
    assert round(float(got["c"].sum()), 5) == 5.39896


def test_reference_known_answers_layernorm(hip):
    """tests/layernorm_test.py:19-22 of the reference; exercises the
    lockstep path (the output reuses the arena slot of 1/sqrt(var))."""
    from ad_amd.nn import LayerNorm
    x = Tensor(np.array([[5.0, 6.0, 3.0], [4.0, 5.0, 6.0]]), requires_grad=True)
    ln = LayerNorm(3)
    res = ln(x)
    res.backward()
    got = {}
    Receiver(lambda a, b, c: got.update(y=a.copy(), db=b.copy(), ds=c.copy()),
             [res, ln.bias.grad().contigious(), ln.scale.grad().contigious()])
    ad.execute(device=hip())
    assert round(float(got["y"].flatten()[0]), 4) == 0.2673
    assert round(float(got["db"].flatten()[0]), 4) == 2.0
    assert round(float(got["ds"].flatten()[0]), 4) == -0.9575


def test_reference_known_answers_concat_pow2(hip):
    """tests/concat_test.py:28-34 and powtwo_test.py:18-27: exact values."""
    x = Tensor(np.array([[5.0, 6.0, 3.0, 1.0], [4.0, 5.0, 6.0, 3.0]]), requires_grad=True)
    y = Tensor(np.array([[8.0, 9.0, 3.0, 6.0], [3.0, 5.0, 4.0, 2.0]]), requires_grad=True)
    res = ad.concat([x * 2, y * 3], 1).contigious()
    res.backward()
    sq = x.pow2()
    got = {}
    Receiver(lambda r, xg, yg, s: got.update(r=r.copy(), xg=xg.copy(), yg=yg.copy(), s=s.copy()),
             [res, x.grad(), y.grad(), sq])
    ad.execute(device=hip())
    assert np.array_equal(got["r"], np.array([[10, 12, 6, 2, 24, 27, 9, 18], [8, 10, 12, 6, 9, 15, 12, 6]]))
    assert got["xg"].sum() == 16 and got["yg"].sum() == 24
    assert np.array_equal(got["s"], np.array([[25, 36, 9, 1], [16, 25, 36, 9]]))


def test_reference_known_answer_temp_read_through_permute(hip):
    """The reference's temp-access rule (karg.py:47-48) by hand: a fused
    temp read through a transpose yields the element's own value, so
    ``(x*2).T() * 1`` of x = arange(16) as 4x4 gives 2*x, bit-exact (the
    oracle's check of the same answer is in test_oracle.py)."""
    from .test_oracle import TEMP_QUIRK_ANSWER, _temp_through_permute_program
    got = _temp_through_permute_program()
    ad.execute(device=hip())
    assert np.array_equal(got["v"], TEMP_QUIRK_ANSWER)


def test_mlp_parity(hip):
    """examples/linear.py (config 1) for 3 SGD steps: every parameter."""
    a, b = run_both(lambda: programs.mlp(steps=3), hip)
    assert_params_close(a, b)


def test_layernorm_training_parity(hip):
    a, b = run_both(lambda: programs.layernorm_step(rows=8, cols=16, steps=3), hip)
    assert_params_close(a, b)


def test_transformer_parity(hip):
    a, b = run_both(lambda: programs.transformer(layers=1, d_model=32, heads=4, ff=64, seq=4, steps=2), hip)
    assert_params_close(a, b)


def test_batched_transformer_parity(hip):
    """Two sequences per batch (per-sample attention on Index slices, rows
    concatenated back): exercises commands split into several passes where
    the arena reuses a slot inside a fused group."""
    from ad_amd import workloads
    a, b = run_both(lambda: workloads.transformer(layers=2, d_model=32, heads=4, ff=64, seq=8, batch=2,
                                                  steps=2), hip)
    assert_params_close(a, b)


def test_eager_lanes_parity(hip):
    """Uncaptured run with launch groups spread over four streams (each
    cross-stream dependency an event wait) against the oracle."""
    from ad_amd import workloads
    a, b = run_both(lambda: workloads.transformer(layers=2, d_model=32, heads=4, ff=64, seq=8, batch=2,
                                                  steps=3), lambda: hip(use_graphs=False, lanes=4))
    assert_params_close(a, b)


def test_layernorm_wide_parity(hip):
    """LayerNorm fwd+bwd at 64 x 1024 (row reductions of 1024 and column
    reductions of 64) for 2 SGD steps on gamma/beta."""
    from ad_amd import workloads
    a, b = run_both(lambda: workloads.layernorm_train(rows=64, cols=1024, steps=2), hip)
    assert_params_close(a, b)


@pytest.mark.parametrize("M,K,N", [(128, 4096, 64), (64, 2048, 64), (1024, 4096, 64), (256, 1024, 256)])
@pytest.mark.parametrize("ta", [False, True])
def test_dotprod_split_k(hip, M, K, N, ta):
    """Few output tiles and a long K: the product is split over K into
    partial products combined in chunk order (then +bias, sigmoid)."""
    from ad_amd.device.hip.codegen import dp_config
    assert dp_config(M, N, K)[2] > 1
    rng = np.random.default_rng(M + K + N)
    a = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    b = rng.standard_normal((K, N)).astype(np.float32)
    bias = rng.standard_normal((N,)).astype(np.float32)
    A = Tensor(a)
    r = ((A.T() if ta else A) @ Tensor(b)) + Tensor(bias)
    got = {}
    Receiver(lambda v: got.setdefault("r", v.copy()), [r])
    ad.execute(device=hip())
    ref = (a.T if ta else a).astype(np.float64) @ b.astype(np.float64) + bias
    bound = 4 * K * np.finfo(np.float32).eps * (np.abs(a).max() * np.abs(b).max()) + 1e-5
    np.testing.assert_allclose(got["r"], ref, rtol=0, atol=bound)


def test_dotprod_concat_operands(hip):
    """Operands given as concats (rows of A, columns of B) are gathered into
    dense scratch copies before the MFMA product."""
    from ad_amd.device.hip.codegen import GATHER_MIN_MACS
    rng = np.random.default_rng(7)
    parts_a = [rng.standard_normal((128, 256)).astype(np.float32) for _ in range(3)]
    parts_b = [rng.standard_normal((256, 64)).astype(np.float32) for _ in range(2)]
    A = ad.concat([Tensor(x) for x in parts_a], 0)
    B = ad.concat([Tensor(x) for x in parts_b], 1)
    assert 384 * 256 * 128 >= GATHER_MIN_MACS
    r = A @ B
    got = {}
    Receiver(lambda v: got.setdefault("r", v.copy()), [r])
    ad.execute(device=hip())
    a = np.concatenate(parts_a, 0).astype(np.float64)
    b = np.concatenate(parts_b, 1).astype(np.float64)
    bound = 4 * 256 * np.finfo(np.float32).eps * (np.abs(a).max() * np.abs(b).max())
    np.testing.assert_allclose(got["r"], a @ b, rtol=0, atol=bound)


@pytest.mark.parametrize("ragged", [False, True])
def test_dotprod_concat_of_transposed_pieces(hip, ragged):
    """Operands whose concat pieces run along the product's rows (transposed
    pieces, concatenated along K for A and along K for B) are gathered
    column-major, reading every piece in order; the product reads the copy
    along its contiguous axis.  Ragged: piece widths and M not multiples of
    4 (a scalar gather)."""
    from ad_amd.device.hip import codegen
    rng = np.random.default_rng(11 + ragged)
    M, N = (257, 130) if ragged else (256, 128)
    ka = [61, 67, 128] if ragged else [64, 64, 128]
    pa = [rng.standard_normal((k, M)).astype(np.float32) for k in ka]        # piece^T is [M, k]
    pb = [rng.standard_normal((N, k)).astype(np.float32) for k in ka]        # piece^T is [k, N]
    A = ad.concat([Tensor(x).T() for x in pa], 1)
    B = ad.concat([Tensor(x).T() for x in pb], 0)
    K = sum(ka)
    assert M * N * K >= codegen.GATHER_MIN_MACS
    r = A @ B
    got = {}
    Receiver(lambda v: got.setdefault("r", v.copy()), [r])
    dev = hip()
    ad.execute(device=dev)
    srcs = [p.source for ps in dev.kernels.values() for p in ps]
    assert sum("_x = _global_id % " in src for src in srcs) == 2, "both operands gathered column-major"
    a = np.concatenate([x.T for x in pa], 1).astype(np.float64)
    b = np.concatenate([x.T for x in pb], 0).astype(np.float64)
    bound = np.sqrt(K) * np.finfo(np.float32).eps * (np.abs(a) @ np.abs(b))
    assert np.all(np.abs(got["r"] - a @ b) <= bound)


@pytest.mark.parametrize("rows,cols", [(4096, 256), (16384, 64), (1000, 100)])
def test_column_reduce_split(hip, rows, cols):
    """Reductions over rows of a row-major matrix (bias / LayerNorm gradient
    shape): split over blocks of rows, combined in order; SUM and MAX."""
    rng = np.random.default_rng(rows + cols)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    X = Tensor(x)
    s = X.sum(0) * 0.5
    m = X.max(0)
    got = {}
    Receiver(lambda a, b: got.update(s=a.copy(), m=b.copy()), [s, m])
    ad.execute(device=hip())
    if rows & (rows - 1) == 0:
        # a power-of-two tree sums every element
        np.testing.assert_allclose(got["s"], 0.5 * x.astype(np.float64).sum(0),
                                   rtol=0, atol=rows * np.finfo(np.float32).eps * 4)
    # otherwise the reference's tree drops elements (and MAX pads with 0):
    # compare with the oracle, which restates that tree
    ad.reset()
    X = Tensor(x)
    s = X.sum(0) * 0.5
    m = X.max(0)
    want = {}
    Receiver(lambda a, b: want.update(s=a.copy(), m=b.copy()), [s, m])
    ad.execute(device=OracleDevice())
    np.testing.assert_allclose(got["s"], want["s"], rtol=1e-4, atol=1e-4)
    assert np.array_equal(got["m"], want["m"])


def test_wide_streamed_sum(hip, monkeypatch):
    """A sum of 20 operands, one element per thread with every operand
    loaded nontemporally (the pass-size threshold lowered to 1 MiB), then
    scaled: against float64, in the reference's left-to-right order."""
    from ad_amd.device.hip import codegen
    monkeypatch.setattr(codegen, "STREAM_PASS_BYTES", 1 << 20)
    rng = np.random.default_rng(20)
    xs = [rng.standard_normal((512, 1024)).astype(np.float32) for _ in range(20)]
    r = Tensor(xs[0])
    for x in xs[1:]:
        r = r + Tensor(x)
    got = {}
    Receiver(lambda v: got.update(r=v.copy()), [r * 0.5])
    dev = hip()
    ad.execute(device=dev)
    assert any("__builtin_nontemporal_load(" in p.source for ps in dev.kernels.values() for p in ps)
    want = np.zeros(xs[0].shape, np.float32)
    for x in xs:
        want = want + x
    np.testing.assert_allclose(got["r"], 0.5 * want, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("rows,cols", [(16387, 256), (8193, 512), (4099, 1024), (16384, 1024)])
def test_row_reduce_ragged_row_counts(hip, rows, cols):
    """Reductions of short contiguous rows over a row count that leaves the
    waves' last pass ragged: SUM against float64 (a power-of-two row sums
    every element), MAX exactly."""
    rng = np.random.default_rng(rows + cols)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    X = Tensor(x)
    got = {}
    Receiver(lambda a, b: got.update(s=a.copy(), m=b.copy()), [X.sum(-1) * 0.5, X.max(-1)])
    ad.execute(device=hip())
    np.testing.assert_allclose(got["s"].reshape(-1), 0.5 * x.astype(np.float64).sum(-1),
                               rtol=0, atol=cols * np.finfo(np.float32).eps * 4)
    assert np.array_equal(got["m"].reshape(-1), x.max(-1))


@pytest.mark.parametrize("iters", [1, 2, 7, 50, 100])
def test_feeder_values_reach_every_iteration(hip, iters):
    """A loop accumulates a value fed by the host each iteration (1, 2, ...):
    the staged copies on the transfer stream must land before, and only
    before, the iteration that reads them -- in graphs of one iteration and
    in unrolled graphs of 32 (50 = 32 + 18 single launches, 100 = 3 x 32 + 4).
    The sum is exact in fp32."""
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
    ad.execute(device=hip())
    assert count[0] == iters
    assert np.all(got["acc"] == iters * (iters + 1) / 2)


@pytest.mark.parametrize("lag", [0, 1])
@pytest.mark.parametrize("iters", [1, 2, 7, 50])
def test_receiver_in_loop_every_iteration(hip, iters, lag):
    """A Receiver inside a replayed loop sees every iteration's value, in
    order: the graph snapshots the data, the transfer stream fetches it, and
    the callback runs ``lag`` iterations later.  Exact in fp32."""
    holder = [Tensor(np.zeros((4, 64), dtype=np.float32))]
    count = [0]
    seen = []

    def feed():
        count[0] += 1
        return np.full((4, 64), float(count[0]), dtype=np.float32)

    def body():
        holder[0] += ad.Feeder(feed, shape=[4, 64])
        Receiver(lambda v: seen.append(v.copy()), [holder[0]])
    ad.ir_for(range(iters), body)
    dev = hip(receiver_lag=lag)
    ad.execute(device=dev)
    assert dev._graphs, "the loop body was not replayed as a graph"
    assert count[0] == iters and len(seen) == iters
    for i, v in enumerate(seen):
        assert np.all(v == (i + 1) * (i + 2) / 2), i


@pytest.mark.parametrize("lag", [0, 1])
def test_logged_training_parity(hip, lag):
    """Per-iteration outputs received inside a replayed training loop, and
    the final parameters, against the oracle."""
    ad.reset()
    a = programs.mlp_logged(steps=6)
    dev = hip(receiver_lag=lag)
    ad.execute(device=dev)
    assert dev._graphs
    ad.reset()
    b = programs.mlp_logged(steps=6)
    ad.execute(device=OracleDevice())
    assert len(a["log"]) == len(b["log"]) == 6
    for x, y in zip(a["log"], b["log"]):
        np.testing.assert_allclose(x, y, rtol=1e-4, atol=1e-5)
    assert_params_close(a, b)


@pytest.mark.parametrize("ta", [False, True])
def test_dotprod_partial_tile_rows(hip, ta):
    """A partial last row of tiles (M = 4160) in a large product."""
    M, K, N = 4160, 256, 4096
    rng = np.random.default_rng(11)
    a = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    b = rng.standard_normal((K, N)).astype(np.float32)
    A = Tensor(a)
    r = (A.T() if ta else A) @ Tensor(b)
    got = {}
    Receiver(lambda v: got.setdefault("r", v.copy()), [r])
    ad.execute(device=hip())
    aa = (a.T if ta else a).astype(np.float64)
    rows = np.concatenate([np.arange(0, 64), np.arange(M - 128, M)])
    ref = aa[rows] @ b.astype(np.float64)
    bound = 4 * K * np.finfo(np.float32).eps * (np.abs(a).max() * np.abs(b).max())
    np.testing.assert_allclose(got["r"][rows], ref, rtol=0, atol=bound)


def test_feeder_offset_zero_matches_the_opencl_oracle(hip):
    """feeder_offset_zero reproduces the OpenCL write_buffer, which puts a
    Feeder at offset 0 of its buffer (cl_helper.py:316,326); the MLP's Feeder
    sits at a non-zero arena offset, so the default differs from it."""
    ad.reset()
    a = programs.mlp(steps=3)
    ad.execute(device=hip(feeder_offset_zero=True))
    ad.reset()
    b = programs.mlp(steps=3)
    ad.execute(device=OracleDevice(feeder_offset_zero=True))
    assert_params_close(a, b)
    ad.reset()
    c = programs.mlp(steps=3)
    ad.execute(device=OracleDevice())
    assert any(not np.allclose(x, y) for x, y in zip(a["params"], c["params"]))


@pytest.mark.parametrize("R", [5, 6, 1000, 1024])
def test_exact_reduce_all_elements(hip, R):
    """exact_reduce: row and column SUM and MAX over every element (the
    reference's tree drops elements for R = 5, 6, 1000 and pads MAX with 0),
    against numpy and the oracle's exact mode."""
    rng = np.random.default_rng(R)
    a = rng.standard_normal((12, R)).astype(np.float32)
    neg = -np.abs(a) - 0.5
    col = rng.standard_normal((R, 12)).astype(np.float32)

    def build(out):
        Receiver(lambda s, m, cs, cm: out.update(s=s.copy(), m=m.copy(), cs=cs.copy(), cm=cm.copy()),
                 [Tensor(a).sum(-1), Tensor(neg).max(-1), Tensor(col).sum(0), Tensor(-np.abs(col) - 0.5).max(0)])
    ad.reset()
    got = {}
    build(got)
    ad.execute(device=hip(exact_reduce=True))
    ad.reset()
    ref = {}
    build(ref)
    ad.execute(device=OracleDevice(exact_reduce=True))
    np.testing.assert_allclose(got["s"], a.astype(np.float64).sum(-1), rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(got["cs"], col.astype(np.float64).sum(0), rtol=1e-5, atol=1e-4)
    assert np.array_equal(got["m"], neg.max(-1))
    assert np.array_equal(got["cm"], (-np.abs(col) - 0.5).max(0))
    for k in got:
        np.testing.assert_allclose(got[k].reshape(-1), ref[k].reshape(-1), rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("M,K,N", [(256, 512, 128), (300, 200, 130), (1, 3, 1), (130, 70, 257), (64, 4096, 64),
                                   (520, 1024, 300)])
@pytest.mark.parametrize("ta,tb", [(False, False), (True, True)])
def test_bf16_dotprod_bound(hip, M, K, N, ta, tb):
    """dot_precision="bf16" (beyond the reference): operands rounded to
    bfloat16 (unit roundoff 2^-8), products exact in fp32, fp32 sums.  Each
    output obeys |C - A@B| <= (2^-7 + 2^-15 + K 2^-23) (|A| @ |B|), against
    float64; the epilogue (+bias) runs on the product as in fp32."""
    rng = np.random.default_rng(M * 13 + K * 5 + N)
    a = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    b = rng.standard_normal((N, K) if tb else (K, N)).astype(np.float32)
    bias = rng.standard_normal((N,)).astype(np.float32)
    r = ((Tensor(a).T() if ta else Tensor(a)) @ (Tensor(b).T() if tb else Tensor(b))) + Tensor(bias)
    got = {}
    Receiver(lambda v: got.setdefault("r", v.copy()), [r])
    ad.execute(device=hip(dot_precision="bf16", bf16_min_macs=0))
    aa = (a.T if ta else a).astype(np.float64)
    bb = (b.T if tb else b).astype(np.float64)
    ref = aa @ bb + bias
    bound = (2.0 ** -7 + 2.0 ** -15 + K * 2.0 ** -23) * (np.abs(aa) @ np.abs(bb)) + 1e-6
    err = np.abs(got["r"] - ref)
    assert np.all(err <= bound), float((err / bound).max())
    if K > 16:
        # the rounding is really there: fp32 operands would be far closer
        assert err.max() > 1e-4 * np.abs(ref).max()


def test_bf16_training_steps(hip):
    """A transformer trained for 3 steps with bf16 DotProds stays close to
    the fp32 oracle (parameters move by lr * grad; the bf16 gradients differ
    by about 1 %)."""
    from ad_amd import workloads
    a, b = run_both(lambda: workloads.transformer(layers=1, d_model=64, heads=4, ff=128, seq=16, batch=2,
                                                  steps=3), lambda: hip(dot_precision="bf16", bf16_min_macs=0))
    for x, y in zip(a["params"], b["params"]):
        assert np.all(np.isfinite(x))
        np.testing.assert_allclose(x, y, rtol=0, atol=2e-3)


def test_bf16_leaves_small_products_fp32(hip):
    """Under dot_precision="bf16", DotProds below bf16_min_macs run the fp32
    kernel: the result equals the fp32 backend's bit for bit."""
    rng = np.random.default_rng(5)
    a = rng.standard_normal((256, 256)).astype(np.float32)
    b = rng.standard_normal((256, 256)).astype(np.float32)
    out = []
    for dev in (hip(dot_precision="bf16"), hip()):
        ad.reset()
        got = {}
        Receiver(lambda v: got.setdefault("r", v.copy()), [Tensor(a) @ Tensor(b)])
        ad.execute(device=dev)
        out.append(got["r"])
    assert np.array_equal(out[0], out[1])


def test_many_piece_concat_reads_arguments_lazily(hip):
    """A concat of 40 row blocks (a kernel with more table arguments than it
    loads at entry) and a DotProd on it, against the oracle."""
    def build():
        rng = np.random.default_rng(5)
        parts = [Tensor(rng.standard_normal((4, 8)).astype(np.float32)) for _ in range(40)]
        w = Tensor(rng.standard_normal((8, 16)).astype(np.float32))
        got = {}
        c = ad.concat(parts, 0)
        Receiver(lambda a, b: got.update(c=a.copy(), p=b.copy()), [(c * 1.5).contigious(), c @ w])
        return got
    ad.reset()
    a = build()
    ad.execute(device=hip())
    ad.reset()
    b = build()
    ad.execute(device=OracleDevice())
    assert np.array_equal(a["c"], b["c"])
    np.testing.assert_allclose(a["p"], b["p"], rtol=1e-4, atol=1e-5)


def test_short_heavy_pass_matches_oracle(hip):
    """A 2^18-element chain of 15 statements (one element per thread)."""
    def build():
        rng = np.random.default_rng(6)
        x = Tensor(rng.standard_normal((1 << 18,)).astype(np.float32))
        y = x * 0.5
        for _ in range(7):
            y = y * 0.75 + x
        got = {}
        Receiver(lambda v: got.update(y=v.copy()), [y])
        return got
    ad.reset()
    a = build()
    ad.execute(device=hip())
    ad.reset()
    b = build()
    ad.execute(device=OracleDevice())
    np.testing.assert_allclose(a["y"], b["y"], rtol=1e-5, atol=1e-6)


def test_heavy_pass_prefetch_batches_match_oracle(hip):
    """A 2^16-element pass reading 70 inputs (more than one prefetch batch
    of operand reads), a concat operand, the same input read by several
    statements, and partial results stored and read back by later
    statements of the same pass: the reads issued ahead in batches give the
    oracle's values."""
    from ad_amd.device.hip import codegen

    def build():
        rng = np.random.default_rng(8)
        xs = [Tensor(rng.standard_normal((256, 256)).astype(np.float32)) for _ in range(70)]
        c = ad.concat([xs[0][:128] * 2.0, xs[1][128:] * 3.0], 0)
        y = c * xs[2]
        parts = []
        for i, x in enumerate(xs[3:]):
            y = y * 0.5 + x * xs[i % 7]
            if i in (20, 45, 66):
                parts.append(y * 1.5)
        got = {}
        Receiver(lambda *v: got.update(v=[a.copy() for a in v]), parts)
        return got
    ad.reset()
    a = build()
    dev = hip()
    ad.execute(device=dev)
    srcs = [p.source for ps in dev.kernels.values() for p in ps]
    assert any(src.count("__builtin_amdgcn_sched_barrier(0)") >= 2 for src in srcs), "no batched pass"
    ad.reset()
    b = build()
    ad.execute(device=OracleDevice())
    for x, y in zip(a["v"], b["v"]):
        np.testing.assert_allclose(x, y, rtol=1e-5, atol=1e-6)
    assert codegen.PREFETCH_BATCH < 70


def test_wide_sum_of_many_operands_matches_oracle(hip):
    """A 2^20-element sum of 20 inputs with a broadcast row factor and two
    stored partial sums (one element per thread, many operands)."""
    def build():
        rng = np.random.default_rng(7)
        xs = [Tensor(rng.standard_normal((1024, 1024)).astype(np.float32)) for _ in range(20)]
        w = Tensor(rng.standard_normal((1024,)).astype(np.float32))
        y = xs[0]
        parts = []
        for i, x in enumerate(xs[1:]):
            y = y + x
            if i in (9, 18):
                parts.append(y * w)
        got = {}
        Receiver(lambda *v: got.update(v=[a.copy() for a in v]), parts)
        return got
    ad.reset()
    a = build()
    ad.execute(device=hip())
    ad.reset()
    b = build()
    ad.execute(device=OracleDevice())
    for u, v in zip(a["v"], b["v"]):
        np.testing.assert_allclose(u, v, rtol=1e-5, atol=1e-5)


def test_skinny_dotprod_epilogue_and_training(hip):
    """Products of at most 8 rows (the skinny kernel) with fused epilogues:
    the C1 MLP (rows of 2) trained 5 steps against the oracle, and
    sigmoid(A @ B + bias) on [5, 300] x [300, 70] against the oracle."""
    a, b = run_both(lambda: programs.mlp(steps=5), hip)
    assert_params_close(a, b)

    def build():
        rng = np.random.default_rng(11)
        x = Tensor(rng.standard_normal((5, 300)).astype(np.float32))
        w = Tensor(rng.standard_normal((300, 70)).astype(np.float32) * 0.05)
        bias = Tensor(rng.standard_normal((70,)).astype(np.float32))
        got = {}
        Receiver(lambda v: got.update(y=v.copy()), [((x @ w) + bias).sigmoid()])
        return got
    ad.reset()
    g = build()
    ad.execute(device=hip())
    ad.reset()
    w = build()
    ad.execute(device=OracleDevice())
    np.testing.assert_allclose(g["y"], w["y"], rtol=1e-4, atol=1e-5)


def test_feeder_after_receiver_runs_command_by_command(hip):
    """A loop body that receives a value and then feeds the next one cannot
    be replayed as a graph (the host callback must run between them): it
    runs command by command, in the reference's order, and every iteration's
    received value matches the oracle's (exact in fp32)."""
    def build():
        acc = [Tensor(np.zeros((4, 8), np.float32))]
        seen = []
        count = [0]

        def feed():
            count[0] += 1
            return np.full((4, 8), float(count[0]), np.float32)

        def body():
            Receiver(lambda v: seen.append(v.copy()), [acc[0]])
            acc[0] += ad.Feeder(feed, shape=[4, 8])
        ad.ir_for(range(5), body)
        return seen
    ad.reset()
    got = build()
    dev = hip()
    ad.execute(device=dev)
    assert not dev._graphs
    ad.reset()
    want = build()
    ad.execute(device=OracleDevice())
    assert len(got) == len(want) == 5
    for x, y in zip(got, want):
        assert np.array_equal(x, y)


@pytest.mark.parametrize("rows,cols,op", [(16384, 1024, 0), (3000, 100, 1), (5, 7, 0), (64, 4096, 1)])
def test_library_column_reduction(rows, cols, op):
    """adhip_reduce_cols (the C ABI's column SUM / MAX over device memory)
    against float64 numpy: sums within a sqrt(rows)-scaled bound, maxima
    exact."""
    from ad_amd.device.hip.runtime import Context
    ctx = Context(0)
    try:
        x = np.random.default_rng(rows + cols).standard_normal((rows, cols), dtype=np.float32)
        out_off = 4 * rows * cols + 256
        ctx.reserve(out_off + 4 * cols + 256)
        ctx.write(0, x)
        ctx.reduce_cols(0, out_off, rows, cols, op)
        got = np.empty(cols, np.float32)
        ctx.read(out_off, got)
    finally:
        ctx.close()
    if op == 0:
        want = x.astype(np.float64).sum(0)
        bound = np.sqrt(rows) * 4 * np.finfo(np.float32).eps * np.abs(x).astype(np.float64).sum(0)
        assert np.all(np.abs(got - want) <= bound)
    else:
        assert np.array_equal(got, x.max(0))
