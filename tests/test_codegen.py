"""Static analyses of the HIP code generator, checked by brute force, and
the C ABI of libadhip.so (loads and exports what include/adhip.h declares;
no device calls)."""
import ctypes
import pathlib
import re

import numpy as np
import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

from ad_amd.device.hip import analysis, codegen
from ad_amd.expr import (Add, BitwiseAnd, Constant, Div, Global, MoreThan, Mult, Remainder,
                         ShiftLeft, ShiftRight, Val, X, Y, evaluate)

ROOT = pathlib.Path(__file__).resolve().parents[1]


def C(v):
    return Val(Constant(v))


@st.composite
def exprs(draw, depth=3, leaves=(Global,)):
    if depth == 0 or draw(st.integers(0, 3)) == 0:
        if draw(st.booleans()):
            return draw(st.sampled_from(leaves))()
        return C(draw(st.integers(0, 40)))
    op = draw(st.sampled_from(["add", "mul", "shl", "shr", "div", "mod", "and", "gt"]))
    a = draw(exprs(depth - 1, leaves))
    k = draw(st.integers(1, 12))
    if op == "add":
        return Add(a, draw(exprs(depth - 1, leaves)))
    if op == "mul":
        return Mult(a, C(k))
    if op == "shl":
        return ShiftLeft(a, C(k % 5))
    if op == "shr":
        return ShiftRight(a, C(k % 5))
    if op == "div":
        return Div(a, C(k))
    if op == "mod":
        return Remainder(a, C(k))
    if op == "and":
        return BitwiseAnd(a, C(k * 5))
    return MoreThan(a, C(k))


@settings(max_examples=300, deadline=None)
@given(exprs())
def test_split_const_preserves_value(e):
    core, c = analysis.split_const(e)
    for g in range(64):
        assert evaluate(core, g=g) + c == evaluate(e, g=g)


@settings(max_examples=300, deadline=None)
@given(exprs())
def test_upper_bound_is_sound(e):
    ub = analysis.upper_bound(e, gmax=63)
    assert max(evaluate(e, g=g) for g in range(64)) <= ub


@settings(max_examples=500, deadline=None)
@given(exprs(depth=4))
def test_vec_class_is_sound(e):
    """AFF: f(4t+i) == f(4t)+i (and f(4t) % 4 == 0 when aligned);
    INV: f(4t+i) == f(4t), over every aligned group."""
    vc = analysis.vec_class(e, Global)
    for t in range(0, 256, 4):
        base = evaluate(e, g=t)
        for i in range(4):
            v = evaluate(e, g=t + i)
            if vc.kind == analysis.AFF:
                assert v == base + i
            elif vc.kind == analysis.INV:
                assert v == base
        if vc.kind == analysis.AFF and vc.al:
            assert base % 4 == 0
        if vc.kind == analysis.INV and vc.al:
            assert base % 4 == 0


@settings(max_examples=300, deadline=None)
@given(exprs(depth=3, leaves=(X, Y)))
def test_vec_class_other_axis_is_invariant(e):
    """Classifying along Y treats X as fixed within a group."""
    vc = analysis.vec_class(e, Y)
    for x in (0, 3, 7):
        for t in range(0, 64, 4):
            base = evaluate(e, x=x, y=t)
            for i in range(4):
                v = evaluate(e, x=x, y=t + i)
                if vc.kind == analysis.AFF:
                    assert v == base + i
                elif vc.kind == analysis.INV:
                    assert v == base


@pytest.mark.parametrize("r", list(range(1, 40)) + [255, 256, 1000, 1024])
def test_tree_inclusion_matches_simulation(r):
    """codegen.tree_inclusion == the reference tree (reduce.py:33-43) run on
    one-hot rows."""
    L = -(-r // 2) * 2
    inc = set(codegen.tree_inclusion(r))
    for y in range(L):
        s = [0.0] * L
        s[y] = 1.0
        off = L // 2
        while off > 0:
            for j in range(off):
                s[j] += s[j + off]
            off >>= 1
        assert (s[0] == 1.0) == (y in inc)


def test_library_exports_header_symbols():
    """libadhip.so loads and exports every function include/adhip.h declares."""
    header = (ROOT / "include" / "adhip.h").read_text()
    names = set(re.findall(r"\b(adhip_[a-z_]+)\s*\(", header))
    lib = ctypes.CDLL(str(ROOT / "ad_amd" / "device" / "hip" / "libadhip.so"))
    missing = [n for n in sorted(names) if not hasattr(lib, n)]
    assert not missing, missing
    from ad_amd.device.hip import runtime
    assert names == set(runtime.EXPORTS)


def test_generated_kernels_compile_for_gfx950():
    """Every kernel of the MLP and LayerNorm programs compiles through
    hipRTC for gfx950 (no device needed)."""
    import ad_amd as ad
    from ad_amd.alloc import AllocEntry
    from ad_amd.fusion import FuseBase
    from ad_amd.graph import Feeder, ForNode, Receiver
    from ad_amd.node import Node
    from ad_amd.device.hip.runtime import HEADER_PATH, compile_source
    from . import programs
    programs.mlp(steps=1)
    proc = ad.compile_proc()
    allocs, cmds = [], []

    def walk(p):
        for c in p.procedure:
            if isinstance(c, ForNode):
                walk(c.get_proc())
            elif isinstance(c, AllocEntry):
                allocs.append(c)
            elif isinstance(c, (Node, FuseBase)) and not isinstance(c, (Feeder, Receiver)):
                cmds.append(c)
    walk(proc)
    info = codegen.BufferInfo()
    for a in allocs:
        info.size[a.id] = a.size
    header = pathlib.Path(HEADER_PATH).read_text()
    for c in cmds:
        for plan in codegen.command_plans(c, info, 0)[0]:
            assert len(compile_source(header + plan.source)) > 0


# ---------------------------------------------------------------- components
class _Stmt:
    def __init__(self, kargs, kres):
        self.kargs, self.kres = kargs, kres


class _Decl:
    def __init__(self, i):
        self.id = i


def _km(i, temp=False, var=None):
    from ad_amd.expr import Global
    from ad_amd.kernalize import KMatrix
    k = KMatrix(i, Global(), [1])
    k.is_temp = temp
    if var is not None:
        k.tetris_var = var
    return k


@pytest.mark.parametrize("seed", range(60))
def test_components_keep_linked_statements_together(seed):
    """Statements sharing a temp, or touching overlapping ranges with at
    least one write, end up in one group; groups keep statement order."""
    import random
    from ad_amd.device.hip import codegen
    rng = random.Random(seed)
    info = codegen.BufferInfo()
    info.size = {1: 100, 2: 100}
    stmts, temps = [], []
    for i in range(rng.randint(1, 30)):
        def opnd():
            if rng.random() < 0.3 and temps:
                return _km(rng.choice(temps), temp=True)
            return _km(rng.choice([1, 1, 2]), var=(rng.randint(0, 99), rng.randint(0, 90), rng.randint(1, 10)))
        kargs = [opnd() for _ in range(rng.randint(1, 2))]
        if rng.random() < 0.4:
            t = 1000 + i
            temps.append(t)
            stmts.append(("tmp", _Decl(t)))
            kres = _km(t, temp=True)
        else:
            kres = _km(rng.choice([1, 2]), var=(rng.randint(0, 99), rng.randint(0, 90), rng.randint(1, 10)))
        stmts.append(("bin", _Stmt(kargs, kres)))
    groups = codegen.components(stmts, info)
    gid = {id(st): g for g, grp in enumerate(groups) for st in grp}
    assert len(gid) == len(stmts)

    def acc(st):
        kind, n = st
        if kind == "tmp":
            return [], [], {n.id}
        rs, ws, ts = [], [], set()
        for a in n.kargs:
            (ts.add(a.id) if a.is_temp else rs.append(codegen._region(a, info)[0]))
        (ts.add(n.kres.id) if n.kres.is_temp else ws.append(codegen._region(n.kres, info)[0]))
        return rs, ws, ts

    def ov(p, q):
        return p[0] == q[0] and max(p[1], q[1]) < min(p[2], q[2])
    for a in stmts:
        for b in stmts:
            if a is b:
                continue
            ra, wa, ta = acc(a)
            rb, wb, tb = acc(b)
            if (ta & tb) or any(ov(x, y) for x in wa for y in rb + wb) or any(ov(x, y) for x in wb for y in ra):
                assert gid[id(a)] == gid[id(b)]
    pos = {id(st): i for i, st in enumerate(stmts)}
    for grp in groups:
        idx = [pos[id(st)] for st in grp]
        assert idx == sorted(idx)


@settings(max_examples=300, deadline=None)
@given(exprs(depth=3, leaves=(Global, X, Y)))
def test_vec_class_two_moving_variables_is_sound(e):
    """In a DotProd element space with rows of 64 (g = 64x + y), X is
    constant and Global, Y advance inside aligned groups of 4: AFF means
    f(4t+i) = f(4t) + i and INV means f(4t+i) = f(4t)."""
    vc = analysis.vec_class(e, (Global, Y))
    for x in (0, 1, 5):
        for t in range(0, 64, 4):
            base = evaluate(e, g=64 * x + t, x=x, y=t)
            for i in range(4):
                v = evaluate(e, g=64 * x + t + i, x=x, y=t + i)
                if vc.kind == analysis.AFF:
                    assert v == base + i
                elif vc.kind == analysis.INV:
                    assert v == base
            if vc.kind == analysis.AFF and vc.al:
                assert base % 4 == 0


def test_combine_passes_follow_a_partial_store():
    """Every elementwise pass that combines stored products or partial
    reductions comes right after the pass that stores them, into the same
    scratch location (a missing store would leave the combine reading stale
    scratch)."""
    import ad_amd as ad
    from ad_amd import workloads
    from ad_amd.alloc import AllocEntry
    from ad_amd.graph import ForNode
    ad.reset()
    workloads.transformer(layers=1, d_model=64, heads=4, ff=64, seq=8, batch=2, steps=1, receive=False)
    proc = ad.compile_proc()
    info = codegen.BufferInfo()

    def note(c, _):
        if isinstance(c, AllocEntry):
            info.size[c.id] = c.size
        return c
    proc.walk(note, step_fused=False, step_proc=True)
    inner = [c for c in proc.procedure if isinstance(c, ForNode)][0].get_proc()
    combines = 0
    for cmd in inner.procedure:
        if type(cmd).__name__ in ("Feeder", "Receiver", "AllocEntry", "DeallocEntry"):
            continue
        plans, _, _ = codegen.command_plans(cmd, info, 0)
        for i, p in enumerate(plans):
            if "_value = *reinterpret_cast<const float4*>" in p.source or "float _value = p" in p.source:
                combines += 1
                prev = plans[i - 1]
                assert prev.family in ("dotprod", "reduce")
                assert re.search(r"[\])] = _v(alue)?;", prev.source), prev.source[-600:]
                slot = [a for a in p.args if a[0] == "scratch"]
                assert any(a in prev.args for a in slot)
    assert combines > 0
    ad.reset()


def test_dotprod_epilogues_load_only_epilogue_operands():
    """The operand registers an in-kernel DotProd epilogue fills before its
    statements hold only what the epilogue statements read: never the
    product's own A and B operands (indexed as the output, they would read
    past those operands)."""
    import ad_amd as ad
    from ad_amd import workloads
    from ad_amd.alloc import AllocEntry
    from ad_amd.fusion import DPElwFuse
    from ad_amd.graph import DotProdNode, ForNode, Receiver, Tensor
    ad.reset()
    workloads.transformer(layers=1, d_model=64, heads=4, ff=64, seq=8, batch=2, steps=1, receive=False)
    rng = np.random.default_rng(0)
    a, b = Tensor(rng.standard_normal((64, 32)).astype(np.float32)), Tensor(rng.standard_normal((32, 64)).astype(np.float32))
    Receiver(lambda v: None, [a @ b])
    proc = ad.compile_proc()
    info = codegen.BufferInfo()

    def note(c, _):
        if isinstance(c, AllocEntry):
            info.size[c.id] = c.size
        return c
    proc.walk(note, step_fused=False, step_proc=True)
    cmds = list(proc.procedure)
    for c in proc.procedure:
        if isinstance(c, ForNode):
            cmds.extend(c.get_proc().procedure)
    checked = 0
    for cmd in cmds:
        if not isinstance(cmd, (DPElwFuse, DotProdNode)):
            continue
        stmts = codegen.statements(cmd.nodes if isinstance(cmd, DPElwFuse) else [cmd])
        for p in codegen.command_plans(cmd, info, 0)[0]:
            if p.family != "dotprod" or "kLoads = " not in p.source:
                continue
            n = int(p.source.split("kLoads = ")[1].split(";")[0])
            assert n <= codegen.epilogue_loads(stmts), p.source
            checked += 1
    assert checked > 0
    ad.reset()


def test_temp_read_through_a_permute_is_reported():
    """The reference reads a fused temp through any access as its own
    element (karg.py:47-48): x*2 read transposed inside one ElwFuse.  The
    check names it; identity reads are not reported."""
    import ad_amd as ad
    from ad_amd.device.hip.device import HIPDevice
    from ad_amd.graph import Receiver, Tensor
    ad.reset()
    x = Tensor(np.arange(16, dtype=np.float32).reshape(4, 4))
    y = Tensor(np.ones((4, 4), dtype=np.float32))
    Receiver(lambda v: None, [((x * 2.0).T() * y).contigious()])
    Receiver(lambda v: None, [(x * 3.0) * y])
    proc = ad.compile_proc()
    fused = [c for c in proc.procedure if hasattr(c, "nodes")]
    found = [codegen.temp_access_violations(codegen.statements(c.nodes), "global") for c in fused]
    assert sum(1 for f in found if f) == 1
    bad = [c for c, f in zip(fused, found) if f][0]
    with pytest.raises(ValueError, match="through the access"):
        HIPDevice._check_temps(bad)
    for c, f in zip(fused, found):
        if not f:
            HIPDevice._check_temps(c)
    ad.reset()


# ---------------------------------------------------------------- argument tables
def _concat_program(pieces):
    """A concat of ``pieces`` row blocks, scaled: one elementwise plan with
    a pointer per piece."""
    import ad_amd as ad
    from ad_amd.alloc import AllocEntry
    from ad_amd.graph import Receiver, Tensor
    ad.reset()
    rng = np.random.default_rng(3)
    parts = [Tensor(rng.standard_normal((4, 8)).astype(np.float32)) for _ in range(pieces)]
    Receiver(lambda v: None, [(ad.concat(parts, 0) * 1.5).contigious()])
    proc = ad.compile_proc()
    info = codegen.BufferInfo()
    for c in proc.procedure:
        if isinstance(c, AllocEntry):
            info.size[c.id] = c.size
    cmds = [c for c in proc.procedure if hasattr(c, "program_id") and type(c).__name__ != "Receiver"]
    return [p for c in cmds for p in codegen.command_plans(c, info, 0)[0]]


def test_table_pointers_are_global_and_many_arguments_are_read_lazily():
    """Table pointers are cast to the global address space; past LAZY_ARGS
    arguments the entry point reads each one where the body uses it (no
    device function taking them all), and the source still compiles."""
    from ad_amd.device.hip.runtime import HEADER_PATH, compile_source
    header = pathlib.Path(HEADER_PATH).read_text()
    few = _concat_program(3)
    many = _concat_program(codegen.LAZY_ARGS + 6)
    src_few = next(p.source for p in few if len(p.args) <= codegen.LAZY_ARGS)
    src_many = next(p.source for p in many if len(p.args) > codegen.LAZY_ARGS)
    for src in (src_few, src_many):
        assert "__attribute__((address_space(1)))" in src
        assert len(compile_source(header + src)) > 0
    assert "_body(" in src_few and "_body(" not in src_many
    # every use of an argument reads the table directly
    assert not re.search(r"\bp\d+\b", src_many.split("tbl_) {", 1)[1])


def test_short_heavy_passes_run_one_element_per_thread():
    """An elementwise pass of at most SCALAR_MAX_N elements with more than
    SCALAR_MIN_STMTS statements runs one element per thread; a light one or
    a long one keeps four."""
    import ad_amd as ad
    from ad_amd.alloc import AllocEntry
    from ad_amd.graph import Receiver, Tensor

    def grid(n, ops):
        ad.reset()
        x = Tensor(np.ones((n,), np.float32))
        y = x * 0.5
        for _ in range(ops - 1):
            y = y * 1.25 + x
        Receiver(lambda v: None, [y])
        proc = ad.compile_proc()
        info = codegen.BufferInfo()
        for c in proc.procedure:
            if isinstance(c, AllocEntry):
                info.size[c.id] = c.size
        cmd = next(c for c in proc.procedure if type(c).__name__ == "ElwFuse")
        (plan,), _, _ = codegen.command_plans(cmd, info, 0)
        return plan.grid[0] * 256
    n = codegen.SCALAR_MAX_N
    assert grid(n, codegen.SCALAR_MIN_STMTS) == n            # threads == elements
    assert grid(n, 2) * 4 == n
    assert grid(4 * n, codegen.SCALAR_MIN_STMTS) * 4 == 4 * n


def test_overwritten_small_operand_is_snapshotted_into_one_pass():
    """The LayerNorm deviation command reads the row means through a
    broadcast and writes the squared deviations over the means' memory
    (tetris reuse): the means are copied to scratch first and the two
    statements share one pass (copy + pass instead of two full passes); the
    snapshot's read comes from scratch and no statement up to it writes the
    means."""
    import ad_amd as ad
    from ad_amd import workloads
    from ad_amd.alloc import AllocEntry
    from ad_amd.graph import ForNode
    ad.reset()
    workloads.layernorm_train(rows=256, cols=64, steps=1, receive=False)
    proc = ad.compile_proc()
    info = codegen.BufferInfo()
    for c in proc.procedure:
        if isinstance(c, AllocEntry):
            info.size[c.id] = c.size
    body = next(c for c in proc.procedure if isinstance(c, ForNode)).get_proc()
    found = False
    for cmd in body.procedure:
        if type(cmd).__name__ != "ElwFuse":
            continue
        stmts = codegen.statements(cmd.nodes)
        pairs = codegen.conflict_pairs(stmts, info, "global")
        snapped = codegen.snapshot_reads(stmts, pairs, info, 0) if pairs else None
        if snapped is None:
            continue
        found = True
        new, copies, used = snapped
        assert codegen.conflict_pairs(new, info, "global") == []
        assert len(copies) == 1 and copies[0].grid[0] * 256 * 4 >= 256 and used >= 256
        (ps, need, _) = codegen.command_plans(cmd, info, 0)
        assert len(ps) == 2 and ps[0].grid[0] < ps[1].grid[0] and need == used
        assert ps[1].grid[0] * 256 * 4 == 256 * 64          # one float4 pass over the elements
    assert found
    # the unpacked arena has no such reuse, hence no snapshot
    info_u = codegen.BufferInfo(unpacked=True)
    info_u.size = info.size
    for cmd in body.procedure:
        if type(cmd).__name__ == "ElwFuse":
            stmts = codegen.statements(cmd.nodes)
            assert codegen.conflict_pairs(stmts, info_u, "global") == []


def test_wide_passes_of_many_operands_run_one_element_per_thread():
    """Beyond SCALAR_MAX_N elements, a pass reading at least
    SCALAR_WIDE_MIN_LOADS distinct operands runs one element per thread (up
    to SCALAR_WIDE_MAX_N elements); one reading fewer keeps four."""
    import ad_amd as ad
    from ad_amd.alloc import AllocEntry
    from ad_amd.graph import Receiver, Tensor

    def plan(n, inputs):
        ad.reset()
        xs = [Tensor(np.ones((n,), np.float32)) for _ in range(inputs)]
        y = xs[0]
        for x in xs[1:]:
            y = y + x
        Receiver(lambda v: None, [y])
        proc = ad.compile_proc()
        info = codegen.BufferInfo()
        for c in proc.procedure:
            if isinstance(c, AllocEntry):
                info.size[c.id] = c.size
        cmd = next(c for c in proc.procedure if type(c).__name__ == "ElwFuse")
        (p,), _, _ = codegen.command_plans(cmd, info, 0)
        return p.grid[0] * 256
    n = 4 * codegen.SCALAR_MAX_N
    many = codegen.SCALAR_WIDE_MIN_LOADS
    assert plan(n, many) == n                                  # threads == elements
    assert plan(n, many - 1) * 4 == n
    assert plan(2 * codegen.SCALAR_WIDE_MAX_N, many) * 4 == 2 * codegen.SCALAR_WIDE_MAX_N


def test_products_of_few_rows_use_the_skinny_kernel():
    """A DotProd of at most SKINNY_M rows compiles to dp_skinny (16 columns
    per block, never split), one of at most DIRECT_K terms to dp_direct,
    others to the MFMA tile."""
    import ad_amd as ad
    from ad_amd.alloc import AllocEntry
    from ad_amd.device.hip.runtime import HEADER_PATH, compile_source
    from ad_amd.graph import Receiver, Tensor
    header = pathlib.Path(HEADER_PATH).read_text()
    for M, K, kernel in ((codegen.SKINNY_M, 4096, "dp_skinny"), (codegen.SKINNY_M + 1, 4096, "dp_mfma"),
                         (300, codegen.DIRECT_K, "dp_direct"), (300, codegen.DIRECT_K + 1, "dp_mfma")):
        ad.reset()
        x = Tensor(np.ones((M, K), np.float32))
        w = Tensor(np.ones((K, 40), np.float32))
        Receiver(lambda v: None, [(x @ w).sigmoid()])
        proc = ad.compile_proc()
        info = codegen.BufferInfo()
        for c in proc.procedure:
            if isinstance(c, AllocEntry):
                info.size[c.id] = c.size
        cmd = next(c for c in proc.procedure if type(c).__name__ == "DPElwFuse")
        plans = codegen.command_plans(cmd, info, 0)[0]
        assert any(kernel in p.source for p in plans)
        if kernel == "dp_skinny":
            assert len(plans) == 1 and plans[0].grid == (3, 1, 1)
        if kernel != "dp_mfma":
            assert len(compile_source(header + plans[0].source)) > 0


@pytest.mark.parametrize("M,K,N", [(4096, 4096, 4096), (300, 200, 130)])
def test_bf16_plans_compile(M, K, N):
    """The bf16 option's plans (two operand packs, then the product on the
    256 x 128 tile or the fp32 tile choice, bounded to two blocks per compute
    unit) compile through hipRTC."""
    import ad_amd as ad
    from ad_amd.alloc import AllocEntry
    from ad_amd.device.hip.runtime import HEADER_PATH, compile_source
    from ad_amd.graph import Receiver, Tensor
    header = pathlib.Path(HEADER_PATH).read_text()
    ad.reset()
    a = Tensor(np.ones((M, K), np.float32))
    b = Tensor(np.ones((K, N), np.float32))
    Receiver(lambda v: None, [(a @ b).sigmoid()])
    proc = ad.compile_proc()
    info = codegen.BufferInfo()
    for c in proc.procedure:
        if isinstance(c, AllocEntry):
            info.size[c.id] = c.size
    cmd = next(c for c in proc.procedure if type(c).__name__ == "DPElwFuse")
    plans = codegen.command_plans(cmd, info, 0, codegen.PlanOptions(dot="bf16", bf16_min_macs=0))[0]
    assert [p.family for p in plans][:2] == ["pack", "pack"]
    product = next(p for p in plans if "dp_bf16" in p.source)
    assert "__launch_bounds__(256, 2)" in product.source
    if M >= 256 and N >= 128:
        assert "dp_bf16<256, 128," in product.source
    for p in plans:
        assert len(compile_source(header + p.source)) > 0


def test_region_of_a_variable_slice_is_its_span():
    """An access of a tetris variable conflicts only over the floats its
    access expression can reach (one head's block of a concatenated result),
    not over the whole variable; ``coarse`` and an access without a span
    give the whole variable; unpacked, the range is relative to the
    variable."""
    from ad_amd.kernalize import KMatrix
    k = KMatrix(7, Add(Global(), Val(Constant(1000 + 256))), [256])
    k.tetris_var = (3, 1000, 1024)
    codegen._note_span(k, (256,))
    assert k.span == (1256, 1512)
    packed, unpacked = codegen.BufferInfo(), codegen.BufferInfo(unpacked=True)
    assert codegen._region(k, packed) == ((7, 1256, 1512), 3)
    assert codegen._region(k, packed, coarse=True) == ((7, 1000, 2024), 3)
    assert codegen._region(k, unpacked) == ((("tv", 3), 256, 512), 3)
    k.span = None
    assert codegen._region(k, packed) == ((7, 1000, 2024), 3)


@pytest.mark.parametrize("pieces", [2, 3, 4, 5, 9, 16, 128])
def test_balanced_concat_selects_the_same_piece(pieces):
    """A left-nested chain of concats (kernalize.make_karg's form: the
    condition of each level is ``e > t`` on the same index, thresholds
    falling) rebuilt as a balanced tree picks the same piece for every
    index, with at most ceil(log2(pieces)) + 1 comparisons; a 2-level
    concat (rows of column chains) balances both levels."""
    import math
    from ad_amd.expr import MoreThan, evaluate
    from ad_amd.kernalize import KConcat, KMatrix

    def chain(e, width, leaf_ids):
        k = KMatrix(leaf_ids[0], Global(), [1])
        for i, lid in enumerate(leaf_ids[1:], start=1):
            k = KConcat(k, KMatrix(lid, Global(), [1]), MoreThan(e, Val(Constant(i * width - 1))), [1])
        return k

    def select(k, g, depth=0):
        if isinstance(k, KConcat):
            hit = evaluate(k.condition, g, 0, 0)
            return select(k.karg_two if hit else k.karg_one, g, depth + 1)
        return k.id, depth

    e = Remainder(Global(), Val(Constant(pieces * 7)))
    orig = chain(e, 7, list(range(pieces)))
    bal = codegen.balance_concat(orig)
    for g in range(pieces * 7 * 2):
        want, _ = select(orig, g)
        got, depth = select(bal, g)
        assert got == want
        if pieces >= codegen.CONCAT_BALANCE_MIN:
            assert depth <= math.ceil(math.log2(pieces)) + 1
    # two levels: rows select one of 3 column chains of `pieces` each
    rows = KConcat(KConcat(chain(e, 7, list(range(100, 100 + pieces))),
                           chain(e, 7, list(range(200, 200 + pieces))),
                           MoreThan(Div(Global(), Val(Constant(1000))), Val(Constant(0))), [1]),
                   chain(e, 7, list(range(300, 300 + pieces))),
                   MoreThan(Div(Global(), Val(Constant(1000))), Val(Constant(1))), [1])
    bal2 = codegen.balance_concat(rows)
    for g in list(range(0, 3000, 13)):
        assert select(bal2, g)[0] == select(rows, g)[0]


def test_narrow_launch_policy():
    """dp_quad alternatives: 64 x 64-tile products with K chunks of at least
    QUAD_MIN_CHUNK terms (64-deep panels below 128 terms), taken by launch
    groups of at most NARROW_MAX_BLOCKS 64 x 64 blocks."""
    from ad_amd.device.hip.codegen import NARROW_MAX_BLOCKS, dp_config, quad_config, use_narrow
    # the C5 per-(sample, head) products and the split per-head weight gradient
    assert quad_config(512, 64, 512, dp_config(512, 64, 512)) == (32, 32, 1, 128)
    assert quad_config(512, 512, 64, dp_config(512, 512, 64)) == (32, 32, 1, 64)
    cfg = dp_config(1024, 64, 4096)
    assert cfg[:3] == (64, 64, 8) and quad_config(1024, 64, 4096, cfg) == (32, 32, 8, 128)
    # 128 x 128 tiles, skinny and direct products get none
    assert quad_config(4096, 4096, 4096, dp_config(4096, 4096, 4096)) is None
    assert quad_config(8, 255, 255, (64, 64, 1, 64)) is None
    assert quad_config(255, 255, 2, (64, 64, 1, 64)) is None
    from types import SimpleNamespace
    plan = SimpleNamespace(grid=(1, 8, 1), narrow=None)       # 8 blocks of 64 x 64 per product
    assert not use_narrow(plan, 1)                            # no alternative
    plan.narrow = SimpleNamespace(grid=(2, 16, 1), narrow=None)
    assert use_narrow(plan, NARROW_MAX_BLOCKS // 8) and not use_narrow(plan, NARROW_MAX_BLOCKS // 8 + 1)
