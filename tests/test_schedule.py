"""The launch scheduler: conflicting launches keep Proc order, launches
merged into one never conflict, and running a Proc's commands in the
scheduled order changes no result (checked on the CPU oracle, bit-exact)."""
import random

import numpy as np
import pytest

import ad_amd as ad
from ad_amd import workloads
from ad_amd.alloc import AllocEntry, DeallocEntry
from ad_amd.device.hip import codegen
from ad_amd.device.hip.schedule import RangeDeps, schedule_dag
from ad_amd.graph import Feeder, ForNode, Receiver
from oracle import OracleDevice


def _conflict(a, b):
    """Two launches conflict when a range one writes overlaps a range the
    other reads or writes."""
    (_, ra, wa), (_, rb, wb) = a, b
    def hit(x, y):
        return any(p[0] == q[0] and max(p[1], q[1]) < min(p[2], q[2]) for p in x for q in y)
    return hit(wa, rb) or hit(wa, wb) or hit(wb, ra)


@pytest.mark.parametrize("seed", range(25))
def test_schedule_keeps_conflicting_launches_in_order(seed):
    rng = random.Random(seed)
    launches = []
    for i in range(rng.randint(1, 60)):
        def rnd():
            out = []
            for _ in range(rng.randint(0, 3)):
                lo = rng.randint(0, 40)
                out.append((rng.choice("ab"), lo, lo + rng.randint(0, 12)))
            return out
        launches.append((rng.choice("xyz"), rnd(), rnd()))
    groups, _ = schedule_dag(launches, group_key=lambda item: item)
    order = [i for g in groups for i in g]
    assert sorted(order) == list(range(len(launches)))
    pos = {i: k for k, i in enumerate(order)}
    group_of = {i: gi for gi, g in enumerate(groups) for i in g}
    for i in range(len(launches)):
        for j in range(i + 1, len(launches)):
            if _conflict(launches[i], launches[j]):
                assert pos[i] < pos[j], (i, j)
                assert group_of[i] != group_of[j]
    for g in groups:
        assert len({launches[i][0] for i in g}) == 1


def test_range_deps_split_segments():
    t = RangeDeps()
    assert t.access(0, [], [("a", 0, 10)]) == set()
    assert t.access(1, [("a", 10, 20)], []) == set()     # touching, not overlapping
    assert t.access(2, [("a", 9, 20)], []) == {0}
    assert t.access(3, [("a", 5, 7)], []) == {0}
    assert t.access(4, [], [("a", 6, 8)]) == {0, 3}      # after the writer and the readers since
    assert t.access(5, [], [("a", 7, 9)]) == {0, 4}
    assert t.access(6, [("b", 0, 100)], [("a", 0, 1)]) == {0}


def _regions(proc):
    info = codegen.BufferInfo()

    def note(c, _):
        if isinstance(c, AllocEntry):
            info.size[c.id] = c.size
        return c
    proc.walk(note, step_fused=False, step_proc=True)
    return info


def _reorder(proc, info):
    """Permute every stretch of kernel commands into the scheduled order."""
    out = [c for c in proc.procedure if isinstance(c, (AllocEntry, DeallocEntry))]
    stretch = []

    def flush():
        if not stretch:
            return
        launches = []
        for cmd in stretch:
            reads, writes = codegen.command_regions(cmd, info)
            launches.append((cmd, reads, writes))
        for g in schedule_dag(launches, group_key=lambda c: None)[0]:
            out.extend(launches[i][0] for i in g)
        stretch.clear()

    moved = 0
    for cmd in proc.procedure:
        if isinstance(cmd, (AllocEntry, DeallocEntry)):
            continue
        if isinstance(cmd, (Feeder, Receiver, ForNode)):
            flush()
            out.append(cmd)
            if isinstance(cmd, ForNode):
                moved += _reorder(cmd.get_proc(), info)
            continue
        stretch.append(cmd)
    flush()
    moved += sum(1 for a, b in zip(out, proc.procedure) if a is not b)
    proc.procedure = out
    return moved


@pytest.mark.parametrize("build", ["batched", "layernorm", "mlp"])
def test_scheduled_order_gives_identical_results(build):
    builders = {
        "batched": lambda: workloads.transformer(layers=1, d_model=16, heads=2, ff=16, seq=4, batch=3, steps=2),
        "layernorm": lambda: workloads.layernorm_train(rows=8, cols=16, steps=2),
        "mlp": lambda: workloads.mlp(steps=2, din=16, dh=24, dout=8),
    }
    ad.reset()
    want = builders[build]()
    ad.execute(device=OracleDevice())
    ad.reset()
    got = builders[build]()
    proc = ad.compile_proc()
    moved = _reorder(proc, _regions(proc))
    OracleDevice().execute(proc)
    if build == "batched":
        assert moved > 0          # the schedule really reorders this program
    for a, b in zip(want["params"], got["params"]):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("seed", range(25))
def test_dag_lanes_order_every_conflict(seed):
    """Running the groups on lanes, each lane in order and waiting only for
    the recorded cross-lane dependencies, orders every conflicting pair of
    launches as in program order (checked through the happens-before
    closure of lane order plus waits)."""
    from ad_amd.device.hip.schedule import assign_lanes, schedule_dag
    rng = random.Random(seed)
    launches = []
    for i in range(rng.randint(1, 60)):
        def rnd():
            out = []
            for _ in range(rng.randint(0, 3)):
                lo = rng.randint(0, 40)
                out.append((rng.choice("ab"), lo, lo + rng.randint(0, 12)))
            return out
        launches.append((rng.choice("xyz"), rnd(), rnd()))
    groups, deps = schedule_dag(launches, group_key=lambda item: item)
    lane_of, waits = assign_lanes(deps, 4)
    n = len(groups)
    before = [set() for _ in range(n)]          # groups finished before g starts
    last = {}
    for g in range(n):
        s = lane_of[g]
        preds = set(waits[g])
        if s in last:
            preds.add(last[s])
        for p in preds:
            before[g] |= before[p] | {p}
        last[s] = g
    group_of = {i: g for g, m in enumerate(groups) for i in m}
    for i in range(len(launches)):
        for j in range(i + 1, len(launches)):
            if _conflict(launches[i], launches[j]):
                gi, gj = group_of[i], group_of[j]
                assert gi != gj and gi in before[gj], (i, j)


def test_loop_bodies_with_receivers_are_capturable():
    """A loop body with Receivers replays as a graph (their data is
    snapshotted and fetched); one with a Feeder after a Receiver, or a nested
    loop, runs command by command."""
    from types import SimpleNamespace

    import numpy as np

    import ad_amd as ad
    from ad_amd.device.hip.device import HIPDevice
    from ad_amd.graph import Feeder, ForNode, Receiver, Tensor
    ad.reset()
    t = Tensor(np.zeros((2, 2), dtype=np.float32))
    f = Feeder(lambda: np.zeros((2, 2), np.float32), shape=[2, 2])
    r = Receiver(lambda v: None, [t])
    ok = HIPDevice._capturable
    assert ok(None, SimpleNamespace(procedure=[f, r]))
    assert ok(None, SimpleNamespace(procedure=[r, r]))
    assert not ok(None, SimpleNamespace(procedure=[r, f]))
    loop = ForNode.__new__(ForNode)
    assert not ok(None, SimpleNamespace(procedure=[f, loop]))
    ad.reset()
