"""A fused group under construction (the reference's FuseBase,
autodiff/fusion/base.py:16-89).

A group starts at a node its family accepts as a first member and grows by
one node at a time: a candidate must read something the group already
produces (unless the family fuses unconnected nodes), and it is placed
right after the latest member it may follow.  The members run as one kernel
of the family's template; the group prints as the reference's listings show
it."""
from enum import Enum
from typing import List

from ..node import Node
from .helper import get_deps, get_res

__all__ = ["FuseResult", "FuseBase"]


class FuseResult(Enum):
    INIT = 1          # the node started the group
    ADD = 2           # the node joined the group
    NONE = 3          # the node stays out


def _indented(text: str, pad: str = "    ") -> str:
    return "\n".join(pad + line for line in text.splitlines())


class FuseBase:
    """Families define ``can_start(node)`` and ``can_follow(member, node)``;
    neither may use instance state (the fusion pass asks ``can_start`` of a
    family before creating a group, which draws a fresh id)."""

    def __init__(self, dep_match: bool = True, should_flatten: bool = False):
        from ..context import context
        self.dep_match = dep_match              # a joining node must read the group's results
        self.should_flatten = should_flatten    # keep a foreign group whole when adding it
        self.result_tracker = set()             # ids the members produce
        self.nodes: List[Node] = []
        self.init_node = None
        self.fuse_id = context.get_id()

    def can_start(self, node) -> bool:
        raise NotImplementedError(f"{type(self).__name__} declares no first member")

    def can_follow(self, member, node) -> bool:
        raise NotImplementedError(f"{type(self).__name__} declares no successor rule")

    def _place(self, item, at=None):
        self.result_tracker.update(get_res(item))
        if at is None:
            self.nodes.append(item)
        else:
            self.nodes.insert(at, item)

    def add(self, item, index=None):
        """Add a node, or the members of another group (the group whole when
        ``should_flatten`` and it is of another family)."""
        if isinstance(item, FuseBase) and not (self.should_flatten and type(item) is not type(self)):
            for member in item.nodes:
                self._place(member, index)
        elif isinstance(item, (Node, FuseBase)):
            self._place(item, index)
        else:
            raise TypeError(f"a fused group holds nodes, not {type(item).__name__}")

    def attempt_fuse(self, node, deps=None) -> FuseResult:
        if not self.nodes and self.can_start(node):
            self.init_node = node
            self.add(node)
            return FuseResult.INIT
        reads = get_deps(node) if deps is None else deps
        if self.dep_match and not (self.result_tracker & reads):
            return FuseResult.NONE
        for back, member in enumerate(reversed(self.nodes)):
            if self.can_follow(member, node):
                self.add(node, len(self.nodes) - back)
                return FuseResult.ADD
        return FuseResult.NONE

    def __repr__(self):
        lines = [f"{type(self).__name__} Fusion (fuse_id: {self.fuse_id}):"]
        lines += [_indented(str(n)) for n in self.nodes]
        return "\n".join(lines)
