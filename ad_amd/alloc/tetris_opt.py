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


def place(entries: List[VarEntry]) -> int:
    """Assign ``offset`` to each entry (already sorted largest first);
    return the arena high-water mark."""
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


def tetris_opt(proc):
    var_tracker: Dict[int, Dict[int, VarEntry]] = {}
    counter = [0]

    def record(node, proc_id):
        if proc_id not in var_tracker:
            var_tracker[proc_id] = {}
        if isinstance(node, AllocEntry):
            if not node.is_temp and node.content is None:
                var_tracker[proc_id][node.id] = VarEntry(node.id, counter[0], None, node.size)
        elif isinstance(node, DeallocEntry):
            if node.id in var_tracker[proc_id] and not node.is_temp:
                var_tracker[proc_id][node.id].end_idx = counter[0]
        counter[0] += 1
        return node
    proc.walk(record)

    for proc_id in var_tracker:
        var_tracker[proc_id] = {k: v for k, v in var_tracker[proc_id].items() if v.end_idx is not None}
    by_proc = {proc_id: list(sorted(v.values(), key=lambda x: -x.size))
               for proc_id, v in var_tracker.items() if len(v) > 0}

    max_temp_size = 0
    total_size = 0
    offsetted: Dict[int, List[VarEntry]] = {}
    for proc_id in by_proc:
        total_size += sum(e.size for e in by_proc[proc_id])
        max_temp_size = max(max_temp_size, place(by_proc[proc_id]))
        offsetted[proc_id] = by_proc[proc_id]

    temp_id = context.get_id()
    stats["used"], stats["total"] = max_temp_size, total_size

    def replace_to_temp(node, proc_id):
        if proc_id not in offsetted:
            return node
        entries = offsetted[proc_id]
        if isinstance(node, (AllocEntry, DeallocEntry)):
            for entry in entries:
                if entry.var_id == node.id:
                    return None
        if not isinstance(node, Node):
            return node
        for idx in range(len(node.kargs)):
            for entry in entries:
                _tag(node.kargs[idx], entry)
                node.kargs[idx].rename(entry.var_id, temp_id, _add_offset(entry.offset))
        for entry in entries:
            if not node.kres.is_none():
                _tag(node.kres, entry)
                node.kres.rename(entry.var_id, temp_id, _add_offset(entry.offset))
        return node
    proc.walk(replace_to_temp)

    if max_temp_size > 0:
        proc.insert(0, AllocEntry(temp_id, max_temp_size, content=None))
        proc.append(DeallocEntry(temp_id, max_temp_size))


def _tag(karg, entry):
    """Remember which packed variable (id, offset, size) an operand addresses,
    for the backend's aliasing checks.  Does not change the IR."""
    from ..kernalize import KConcat, KMatrix
    if isinstance(karg, KMatrix):
        if karg.id == entry.var_id:
            karg.tetris_var = (entry.var_id, entry.offset, entry.size)
    elif isinstance(karg, KConcat):
        _tag(karg.karg_one, entry)
        _tag(karg.karg_two, entry)


def _add_offset(offset):
    return lambda expr: simplify_expr(Add(expr, Val(Constant(offset))), None)
