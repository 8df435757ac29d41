"""Launch scheduling for one stretch of a Proc.

The reference runs every command in Proc order on one in-order queue
(autodiff/device/opencl/device.py:114-130).  Commands only interact through
memory, so any order that keeps every pair of launches touching an
overlapping range -- at least one of them writing -- in Proc order gives the
same results.  ``schedule_dag`` assigns each launch a level one past the
highest level of the earlier launches it depends on (read-after-write,
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


class RangeDeps:
    """Per buffer: a partition of the float index line into segments, each
    holding the last launch that wrote it and the launches that read it
    since (the launches a new access must follow)."""

    def __init__(self):
        self._cuts: Dict[object, List[int]] = {}
        self._vals: Dict[object, List[list]] = {}      # [writer, [readers]] per segment

    def _split(self, buf, at):
        cuts = self._cuts.setdefault(buf, [0])
        vals = self._vals.setdefault(buf, [[-1, []]])
        i = bisect_right(cuts, at) - 1
        if cuts[i] != at:
            cuts.insert(i + 1, at)
            vals.insert(i + 1, [vals[i][0], list(vals[i][1])])

    def _segments(self, buf, lo, hi):
        self._split(buf, lo)
        self._split(buf, hi)
        cuts, vals = self._cuts[buf], self._vals[buf]
        return range(bisect_left(cuts, lo), bisect_left(cuts, hi)), vals

    def access(self, me: int, reads: Sequence[Range], writes: Sequence[Range]) -> set:
        """The earlier launches ``me`` must follow; records its accesses."""
        deps = set()
        for buf, lo, hi in reads:
            if hi > lo:
                idx, vals = self._segments(buf, lo, hi)
                for i in idx:
                    if vals[i][0] >= 0:
                        deps.add(vals[i][0])
        for buf, lo, hi in writes:
            if hi > lo:
                idx, vals = self._segments(buf, lo, hi)
                for i in idx:
                    if vals[i][0] >= 0:
                        deps.add(vals[i][0])
                    deps.update(vals[i][1])
        for buf, lo, hi in reads:
            if hi > lo:
                idx, vals = self._segments(buf, lo, hi)
                for i in idx:
                    vals[i][1].append(me)
        for buf, lo, hi in writes:
            if hi > lo:
                idx, vals = self._segments(buf, lo, hi)
                for i in idx:
                    vals[i][0] = me
                    vals[i][1] = []
        deps.discard(me)
        return deps


def schedule_dag(launches: Sequence[Tuple[object, Sequence[Range], Sequence[Range]]],
                 group_key=lambda item: None):
    """As ``schedule``, and also the dependencies between the groups:
    returns ``(groups, deps)`` with ``deps[g]`` the indices of the earlier
    groups group ``g`` must follow (the last writer of every range it reads,
    the last writer and the readers since of every range it writes)."""
    tracker = RangeDeps()
    levels, launch_deps = [], []
    for i, (item, reads, writes) in enumerate(launches):
        d = tracker.access(i, reads, writes)
        launch_deps.append(d)
        levels.append(1 + max((levels[j] for j in d), default=-1))
    by_level: Dict[int, Dict[object, List[int]]] = {}
    for i, (item, _, _) in enumerate(launches):
        key = group_key(item)
        slot = by_level.setdefault(levels[i], {})
        slot.setdefault(key if key is not None else ("solo", i), []).append(i)
    groups = []
    for lvl in sorted(by_level):
        groups.extend(by_level[lvl].values())
    group_of = {i: g for g, members in enumerate(groups) for i in members}
    deps = []
    for g, members in enumerate(groups):
        deps.append(sorted({group_of[j] for i in members for j in launch_deps[i]} - {g}))
    return groups, deps


def assign_lanes(deps: Sequence[Sequence[int]], lanes: int):
    """Give each group (in order) a lane and the waits it needs: a group
    continues the lane whose last group it depends on when there is one,
    otherwise takes the least recently used lane; for every other lane it
    waits only for the latest group it depends on there.  Returns
    ``(lane_of, waits)`` with ``waits[g]`` the groups whose completion group
    ``g`` must wait for across lanes."""
    lane_of, waits = [], []
    tail = [-1] * lanes           # last group on each lane
    used_at = [-1] * lanes        # position of that group, for least-recent choice
    pos_on = {}
    for g, ds in enumerate(deps):
        cont = [s for s in range(lanes) if tail[s] >= 0 and tail[s] in ds]
        s = cont[0] if cont else min(range(lanes), key=lambda k: used_at[k])
        latest = {}
        for d in ds:
            ld = lane_of[d]
            if ld != s and pos_on[d] > latest.get(ld, (-1, None))[0]:
                latest[ld] = (pos_on[d], d)
        lane_of.append(s)
        waits.append(sorted(d for _, d in latest.values()))
        pos_on[g] = g
        tail[s] = g
        used_at[s] = g
    return lane_of, waits
