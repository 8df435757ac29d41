"""The backend on a Proc exactly as the reference's passes leave it.

The reference's tetris pass (alloc/tetris_opt.py:159-188) rewrites every
access of an arena variable to ``expr + offset`` on the shared region and
records nothing else; this repository's restatement additionally notes the
variable on each access (``KMatrix.tetris_var``), which the unpacked arena
uses.  Here every such note is deleted before the device sees the Proc:
the device then derives what each access can touch from the access
expression itself (``codegen.annotate_spans``) and must give the same
results as the oracle, plan a schedule no coarser than with the notes, and
keep every access in bounds."""
import os
import shutil

import numpy as np
import pytest

import ad_amd as ad
from ad_amd import workloads
from ad_amd.device.hip import codegen
from ad_amd.fusion import FuseBase
from ad_amd.graph import ForNode
from oracle import OracleDevice

from .host_emulation import CLANG, check_run, recording_device


def strip_tetris_notes(proc):
    """Delete ``tetris_var`` from every KMatrix of a Proc; returns how many."""
    n = 0

    def walk(p):
        nonlocal n
        for c in p.procedure:
            if isinstance(c, ForNode):
                walk(c.get_proc())
                continue
            for nd in (c.nodes if isinstance(c, FuseBase) else [c]):
                ks = list(getattr(nd, "kargs", []) or [])
                if getattr(nd, "kres", None) is not None:
                    ks.append(nd.kres)
                for k in ks:
                    for km in codegen.iter_kmatrix(k):
                        if hasattr(km, "tetris_var"):
                            del km.tetris_var
                            n += 1
    walk(proc)
    return n


BUILDERS = {
    "mlp": lambda: workloads.mlp(steps=4),
    "layernorm": lambda: workloads.layernorm_train(rows=256, cols=1024, steps=3),
    "transformer": lambda: workloads.transformer(layers=2, d_model=32, heads=4, ff=64, seq=8, batch=2, steps=3),
}


@pytest.mark.parametrize("name", sorted(BUILDERS))
def test_schedule_without_notes_is_no_coarser(name):
    launches = {}
    for stripped in (False, True):
        ad.reset()
        BUILDERS[name]()
        proc = ad.compile_proc()
        if stripped:
            assert strip_tetris_notes(proc) > 0
        dev = recording_device()
        dev.prepare(proc)
        launches[stripped] = dev.stats["launches_per_iter"]
    assert launches[True] <= launches[False]


@pytest.mark.skipif(not os.path.exists(CLANG), reason="needs the ROCm host clang")
@pytest.mark.parametrize("name", sorted(BUILDERS))
def test_program_without_notes_stays_in_bounds(tmp_path, name):
    BUILDERS[name]()
    proc = ad.compile_proc()
    strip_tetris_notes(proc)
    ok, log = check_run(proc, str(tmp_path))
    shutil.rmtree(tmp_path, ignore_errors=True)
    assert ok, log


@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(BUILDERS))
def test_hip_without_notes_matches_oracle(hip, name):
    ad.reset()
    got = BUILDERS[name]()
    proc = ad.compile_proc()
    assert strip_tetris_notes(proc) > 0
    hip().execute(proc)
    ad.reset()
    ref = BUILDERS[name]()
    ad.execute(device=OracleDevice())
    assert len(got["params"]) == len(ref["params"]) > 0
    for x, y in zip(got["params"], ref["params"]):
        np.testing.assert_allclose(x, y, rtol=1e-4, atol=1e-5)
