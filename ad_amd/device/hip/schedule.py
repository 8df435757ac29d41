"""Launch scheduling for one stretch of a Proc.

The reference runs every command in Proc order on one in-order queue
(autodiff/device/opencl/device.py:114-130).  Commands only interact through
memory, so any order that keeps every pair of launches touching an
overlapping range -- at least one of them writing -- in Proc order gives the
same results.  ``schedule`` assigns each launch a level one past the highest
level of any earlier launch it conflicts with (read-after-write,
write-after-read, write-after-write over buffer ranges), then emits the
levels in order; launches of one level share no range written by another,
so launches of one level with the same kernel and launch shape run as ONE
launch (the per-instance arguments come from consecutive rows of an
argument table, indexed by ``blockIdx.z``).

Ranges are ``(buffer, lo, hi)`` in floats: an arena variable's packed
region, a whole Tensor buffer, or the scratch region shared by every
multi-pass command.
"""
from bisect import bisect_left, bisect_right
from typing import Dict, List, Sequence, Tuple

Range = Tuple[object, int, int]


class RangeLevels:
    """Per buffer: a partition of the float index line into segments, each
    holding the highest level that wrote it and that read it so far."""

    def __init__(self):
        self._cuts: Dict[object, List[int]] = {}      # sorted segment starts
        self._vals: Dict[object, List[List[int]]] = {}  # [writer, reader] per segment

    def _split(self, buf, at):
        cuts = self._cuts.setdefault(buf, [0])
        vals = self._vals.setdefault(buf, [[-1, -1]])
        i = bisect_right(cuts, at) - 1
        if cuts[i] != at:
            cuts.insert(i + 1, at)
            vals.insert(i + 1, list(vals[i]))

    def _segments(self, buf, lo, hi):
        self._split(buf, lo)
        self._split(buf, hi)
        cuts, vals = self._cuts[buf], self._vals[buf]
        return range(bisect_left(cuts, lo), bisect_left(cuts, hi)), vals

    def level_for(self, reads: Sequence[Range], writes: Sequence[Range]) -> int:
        lvl = 0
        for buf, lo, hi in reads:
            if hi <= lo:
                continue
            idx, vals = self._segments(buf, lo, hi)
            for i in idx:
                lvl = max(lvl, vals[i][0] + 1)
        for buf, lo, hi in writes:
            if hi <= lo:
                continue
            idx, vals = self._segments(buf, lo, hi)
            for i in idx:
                lvl = max(lvl, vals[i][0] + 1, vals[i][1] + 1)
        return lvl

    def record(self, reads: Sequence[Range], writes: Sequence[Range], lvl: int):
        for buf, lo, hi in reads:
            if hi <= lo:
                continue
            idx, vals = self._segments(buf, lo, hi)
            for i in idx:
                vals[i][1] = max(vals[i][1], lvl)
        for buf, lo, hi in writes:
            if hi <= lo:
                continue
            idx, vals = self._segments(buf, lo, hi)
            for i in idx:
                vals[i][0] = max(vals[i][0], lvl)


def schedule(launches: Sequence[Tuple[object, Sequence[Range], Sequence[Range]]],
             group_key=lambda item: None) -> List[List[int]]:
    """``launches``: ``(item, reads, writes)`` in Proc order.  Returns groups
    of launch indices in execution order; a group holds launches of one level
    whose ``group_key`` is equal and not None (a key of None never groups).
    Within a level, groups appear in the order of their first member."""
    tracker = RangeLevels()
    levels = []
    for item, reads, writes in launches:
        lvl = tracker.level_for(reads, writes)
        tracker.record(reads, writes, lvl)
        levels.append(lvl)
    by_level: Dict[int, Dict[object, List[int]]] = {}
    for i, (item, _, _) in enumerate(launches):
        key = group_key(item)
        slot = by_level.setdefault(levels[i], {})
        slot.setdefault(key if key is not None else ("solo", i), []).append(i)
    out = []
    for lvl in sorted(by_level):
        out.extend(by_level[lvl].values())
    return out
