"""Arena packing ("tetris", autodiff/alloc/tetris_opt.py:69-192).

Per Proc, every non-temp, content-free Alloc with a matching Dealloc is a
rectangle [start, end) x [offset, offset+size) in (command index, float
offset) space.  Largest first (stable), each goes into the LAST gap between
already-placed, lifetime-overlapping ranges that is wide enough, else right
after the last such range; the gap below the lowest range is never used.
All Procs share one arena id; each access to a packed buffer becomes
``simplify(expr + offset)`` on that id."""
from dataclasses import dataclass
from typing import Dict, List, Optional

import numpy as np

from ..context import context
from ..expr import Add, Constant, Val
from ..expr.simplify import simplify_expr
from ..node import Node
from . import AllocEntry, DeallocEntry

stats = {"used": 0, "total": 0}


@dataclass
class VarEntry:
    var_id: int
    start_idx: int
    end_idx: Optional[int]
    size: int
    offset: int = 0


def _lifetimes_overlap(a: VarEntry, b: VarEntry) -> bool:
    return max(a.start_idx, b.start_idx) < min(a.end_idx, b.end_idx)


def _ranges_intersect(r1, r2) -> bool:
    return r1[0] < r2[1] and r2[0] < r1[1]


def _groups_by_sweep(lo, hi):
    """Merged groups of ranges sorted by start, with the pairwise test of
    the reference loop (it matters for empty ranges)."""
    out = []
    for a, b in zip(lo.tolist(), hi.tolist()):
        if out and a < out[-1][1] and out[-1][0] < b:
            out[-1] = (min(out[-1][0], a), max(out[-1][1], b))
        else:
            out.append((a, b))
    return np.array([g[0] for g in out], dtype=np.int64), np.array([g[1] for g in out], dtype=np.int64)


def place(entries: List[VarEntry]) -> int:
    """Assign ``offset`` to each entry (already sorted largest first);
    return the arena high-water mark.

    For each entry: the ranges of already placed entries whose lifetimes
    overlap it, stably sorted by start, intersecting neighbours merged; the
    entry goes into the last gap between consecutive ranges that is wide
    enough, else at the end of the last range, else at 0.  Everything runs
    vectorised over the placed entries: when every range is non-empty, a
    sorted range starts a new merged group exactly when it starts at or
    after the largest end before it, and a group ends at the largest end
    within it (empty ranges take the reference's pairwise sweep)."""
    n = len(entries)
    starts = np.fromiter((e.start_idx for e in entries), dtype=np.int64, count=n)
    ends = np.fromiter((e.end_idx for e in entries), dtype=np.int64, count=n)
    sizes = np.fromiter((e.size for e in entries), dtype=np.int64, count=n)
    offsets = np.zeros(n, dtype=np.int64)
    high = 0
    for i, entry in enumerate(entries):
        live = np.nonzero(np.maximum(starts[:i], starts[i]) < np.minimum(ends[:i], ends[i]))[0]
        if len(live) == 0:
            offset = 0
        else:
            order = np.argsort(offsets[live], kind="stable")     # Python's stable sort by start
            lo = offsets[live][order]
            sz = sizes[live][order]
            if sz.min() > 0:
                reach = np.maximum.accumulate(lo + sz)
                first = np.flatnonzero(lo[1:] >= reach[:-1]) + 1      # ranges that start a group
                group_lo = np.concatenate(([lo[0]], lo[first]))
                group_hi = reach[np.append(first - 1, len(lo) - 1)]
            else:
                group_lo, group_hi = _groups_by_sweep(lo, lo + sz)
            wide = np.flatnonzero(group_lo[1:] - group_hi[:-1] >= entry.size)
            offset = int(group_hi[wide[-1]]) if len(wide) else int(group_hi[-1])
        entry.offset = offset
        offsets[i] = offset
        high = max(high, offset + entry.size)
    return high


def place_reference(entries: List[VarEntry]) -> int:
    """Direct restatement of the placement loop (tetris_opt.py:108-149), one
    lifetime check per placed entry; kept as the check of ``place``."""
    placed: List[VarEntry] = []
    high = 0
    for entry in entries:
        taken = sorted([(o.offset, o.offset + o.size) for o in placed if _lifetimes_overlap(entry, o)],
                       key=lambda r: r[0])
        i = 0
        while i < len(taken) - 1:
            if _ranges_intersect(taken[i], taken[i + 1]):
                merged = (min(taken[i][0], taken[i + 1][0]), max(taken[i][1], taken[i + 1][1]))
                del taken[i]
                del taken[i]
                taken.insert(i, merged)
            else:
                i += 1
        offset = -1
        for t in range(len(taken) - 1):
            if taken[t + 1][0] - taken[t][1] >= entry.size:
                offset = taken[t][1]
        if offset == -1:
            offset = taken[-1][-1] if len(taken) > 0 else 0
        entry.offset = offset
        placed.append(entry)
        high = max(high, offset + entry.size)
    return high


def _lifetimes(proc) -> Dict[int, List[VarEntry]]:
    """Per Proc id: its packable variables -- non-temp, content-free Allocs
    that a non-temp Dealloc of the same Proc closes -- as VarEntry spans
    [Alloc position, Dealloc position) in one count over every command the
    walk visits, largest first (ties keep their first-Alloc order).  A
    variable allocated again restarts its span in place."""
    opened: Dict[int, Dict[int, VarEntry]] = {}
    position = 0

    def note(node, proc_id):
        nonlocal position
        live = opened.setdefault(proc_id, {})
        if isinstance(node, AllocEntry):
            if not node.is_temp and node.content is None:
                live[node.id] = VarEntry(node.id, position, None, node.size)
        elif isinstance(node, DeallocEntry) and not node.is_temp and node.id in live:
            live[node.id].end_idx = position
        position += 1
        return node
    proc.walk(note)
    spans = {}
    for proc_id, live in opened.items():
        closed = [e for e in live.values() if e.end_idx is not None]
        if closed:
            spans[proc_id] = sorted(closed, key=lambda e: -e.size)
    return spans


def tetris_opt(proc):
    by_proc = _lifetimes(proc)

    max_temp_size = 0
    total_size = 0
    offsetted: Dict[int, List[VarEntry]] = {}
    for proc_id in by_proc:
        total_size += sum(e.size for e in by_proc[proc_id])
        max_temp_size = max(max_temp_size, place(by_proc[proc_id]))
        offsetted[proc_id] = by_proc[proc_id]

    temp_id = context.get_id()
    stats["used"], stats["total"] = max_temp_size, total_size

    # One pass: the reference loops over every packed variable for every
    # operand; after its rename an operand carries ``temp_id``, which matches
    # no variable, so a single lookup per operand gives the same result.
    by_var = {proc_id: {e.var_id: e for e in entries} for proc_id, entries in offsetted.items()}

    def relabel(karg, table):
        from ..kernalize import KConcat, KMatrix
        if isinstance(karg, KMatrix):
            entry = table.get(karg.id)
            if entry is not None:
                karg.tetris_var = (entry.var_id, entry.offset, entry.size)
                karg.rename(entry.var_id, temp_id, _add_offset(entry.offset))
        elif isinstance(karg, KConcat):
            relabel(karg.karg_one, table)
            relabel(karg.karg_two, table)

    def replace_to_temp(node, proc_id):
        table = by_var.get(proc_id)
        if table is None:
            return node
        if isinstance(node, (AllocEntry, DeallocEntry)):
            return None if node.id in table else node
        if not isinstance(node, Node):
            return node
        for karg in node.kargs:
            relabel(karg, table)
        if not node.kres.is_none():
            relabel(node.kres, table)
        return node
    proc.walk(replace_to_temp)

    if max_temp_size > 0:
        proc.insert(0, AllocEntry(temp_id, max_temp_size, content=None))
        proc.append(DeallocEntry(temp_id, max_temp_size))


def _add_offset(offset):
    return lambda expr: simplify_expr(Add(expr, Val(Constant(offset))), None)
