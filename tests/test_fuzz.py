"""Random programs (tests/fuzz_programs.py): the oracle against a float64
numpy evaluation of the same program on the CPU, and the HIP backend against
the oracle on the GPU (forward values and input gradients)."""
import numpy as np
import pytest

import ad_amd as ad
from oracle import OracleDevice

from .fuzz_programs import random_program


def _close(x, y, rtol=1e-4):
    scale = max(1.0, float(np.abs(y).max()) if y.size else 1.0)
    np.testing.assert_allclose(x, y, rtol=rtol, atol=rtol * scale)


def _reads_temp_through_permute(proc):
    """The program hits the reference's temp-access quirk (a fused temp read
    through a non-identity access reads the element's own value, karg.py:47-48),
    which the oracle reproduces and plain numpy does not."""
    from ad_amd.device.hip import codegen
    from ad_amd.fusion import DPElwFuse, ReduceElwFuse
    for c in proc.procedure:
        if hasattr(c, "nodes"):
            kind = "dp" if isinstance(c, DPElwFuse) else "red" if isinstance(c, ReduceElwFuse) else "global"
            cols = c.init_node.shape[1] if kind == "dp" else 1
            if codegen.temp_access_violations(codegen.statements(c.nodes), kind, cols):
                return True
    return False


@pytest.mark.parametrize("seed", range(40))
def test_oracle_matches_float64(seed):
    ad.reset()
    got, expected = random_program(seed)
    proc = ad.compile_proc()
    if _reads_temp_through_permute(proc):
        ad.reset()
        pytest.skip("reads a fused temp through a permute (the reference's quirk; numpy differs)")
    OracleDevice().execute(proc)
    assert len(got["outs"]) == len(expected)
    for x, e in zip(got["outs"], expected):
        assert x.shape == e.shape
        _close(x, e)
    ad.reset()


@pytest.mark.gpu
@pytest.mark.parametrize("seed", list(range(30)) + [1000 + s for s in range(20)])
def test_hip_matches_oracle(hip, seed):
    grads = seed >= 1000
    ad.reset()
    got, _ = random_program(seed, grads=grads)
    ad.execute(device=hip())
    ad.reset()
    ref, _ = random_program(seed, grads=grads)
    ad.execute(device=OracleDevice())
    assert len(got["outs"]) == len(ref["outs"])
    for x, y in zip(got["outs"], ref["outs"]):
        assert x.shape == y.shape
        _close(x, y)
    ad.reset()


@pytest.mark.gpu
def test_hip_matches_oracle_concat_in_epilogue(hip):
    """The 12-operation program of seed 2008 with gradients: a DotProd+Elw
    epilogue reads a concat whose piece index underflows outside the
    concat's condition (the piece's load stays inside the conditional)."""
    ad.reset()
    got, _ = random_program(2008, n_ops=12, grads=True)
    ad.execute(device=hip())
    ad.reset()
    ref, _ = random_program(2008, n_ops=12, grads=True)
    ad.execute(device=OracleDevice())
    assert len(got["outs"]) == len(ref["outs"])
    for x, y in zip(got["outs"], ref["outs"]):
        assert x.shape == y.shape
        _close(x, y)
    ad.reset()
