"""Greedy fusion accumulator (autodiff/fusion/base.py:16-89)."""
from enum import Enum
from typing import List

from ..context import indent_str
from ..node import Node
from .helper import get_deps, get_res

__all__ = ["FuseResult", "FuseBase"]


class FuseResult(Enum):
    INIT = 1
    ADD = 2
    NONE = 3


class FuseBase:
    def __init__(self, dep_match=True, should_flatten=False):
        from ..context import context
        self.dep_match = dep_match
        self.should_flatten = should_flatten
        self.result_tracker = set()
        self.nodes: List[Node] = []
        self.init_node = None
        self.fuse_id = context.get_id()

    def _add_node(self, add, index=None):
        for r in get_res(add):
            self.result_tracker.add(r)
        if isinstance(index, int):
            self.nodes.insert(index, add)
        else:
            self.nodes.append(add)

    def add(self, n, index=None):
        if isinstance(n, FuseBase):
            if self.should_flatten and type(self) != type(n):
                self._add_node(n, index)
            else:
                for node in n.nodes:
                    self._add_node(node, index)
        elif isinstance(n, Node):
            self._add_node(n, index)
        else:
            raise TypeError(f"Invalid type: {type(n)}")

    def _fuse(self, node_one, node_two):
        raise NotImplementedError

    def _init(self, node):
        raise NotImplementedError

    def attempt_fuse(self, node, deps=None) -> FuseResult:
        """Start the group with ``node``, or append it right after the last
        member it can follow (fusion/base.py:59-77)."""
        if len(self.nodes) == 0 and self._init(node):
            self.init_node = node
            self.add(node)
            return FuseResult.INIT
        if deps is None:
            deps = get_deps(node)
        if self.dep_match and len(self.result_tracker.intersection(deps)) == 0:
            return FuseResult.NONE
        for idx, n in enumerate(reversed(self.nodes)):
            if self._fuse(n, node):
                self.add(node, len(self.nodes) - idx)
                return FuseResult.ADD
        return FuseResult.NONE

    def __repr__(self):
        out = f"{type(self).__name__} Fusion (fuse_id: {self.fuse_id}):\n"
        for n in self.nodes:
            out += indent_str(str(n)) + "\n"
        return out[:-1]
