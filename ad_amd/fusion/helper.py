"""Dependency and result sets of commands (the behaviour of
autodiff/fusion/helper.py:12-81)."""
from typing import Set

from ..node import Node

__all__ = ["get_deps", "get_res", "get_walking_path"]


def _loop_body(node, step_proc):
    """The Proc of a loop command when loops are stepped into, else None."""
    return node.get_proc() if step_proc and isinstance(node, Node) else None


def get_res(node, step_proc: bool = False) -> Set[int]:
    """Ids a command produces: its own, or everything its loop body (when
    ``step_proc``) or fused group produces."""
    from .base import FuseBase
    if isinstance(node, FuseBase):
        return set().union(*(get_res(member) for member in node.nodes))
    if not isinstance(node, Node):
        raise TypeError(f"get_res: not a command: {type(node).__name__}")
    body = _loop_body(node, step_proc)
    if body is None:
        return {node.id}
    return set().union(*(get_res(cmd, True) for cmd in body.procedure))


def get_deps(node, step_proc: bool = False) -> Set[int]:
    """Ids a command reads.  For a loop (``step_proc``) or fused group: what
    its members read that it does not produce itself."""
    from .base import FuseBase
    if isinstance(node, FuseBase):
        members, produced = node.nodes, get_res(node, step_proc)
    elif isinstance(node, Node):
        body = _loop_body(node, step_proc)
        if body is None:
            return set(node.kargs_child_ids())
        members, produced = body.procedure, get_res(node, True)
    else:
        raise TypeError(f"get_deps: not a command: {type(node).__name__}")
    reads = set()
    for member in members:
        reads.update(d for d in get_deps(member, True) if d not in produced)
    reads.discard(None)
    return reads


def get_walking_path(node, toposort_res, id_to_node) -> Set[int]:
    """``node`` plus every command of the given layers, scanned in order,
    that reads something already on the path."""
    path = {node.id}
    for layer in toposort_res:
        for nid in layer:
            cmd = id_to_node[nid]
            if not path.isdisjoint(get_deps(cmd)):
                path.add(cmd.id)
    return path
