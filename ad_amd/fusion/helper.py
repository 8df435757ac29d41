"""Dependency and result sets of commands (autodiff/fusion/helper.py:12-81)."""
from typing import Set

from ..node import Node

__all__ = ["get_deps", "get_res", "get_walking_path"]


def get_deps(node, step_proc: bool = False) -> Set[int]:
    """Ids a command reads.  For a loop (``step_proc``) or fused group: the
    union over the body minus what the body itself produces."""
    from .base import FuseBase
    if isinstance(node, Node):
        proc = node.get_proc() if step_proc else None
        if proc is not None:
            produced = get_res(node, True)
            out = set()
            for cmd in proc.procedure:
                out.update([d for d in get_deps(cmd, True) if d not in produced])
            return set(filter(lambda x: x is not None, out))
        return set({cid for cid in node.kargs_child_ids()})
    if isinstance(node, FuseBase):
        produced = get_res(node, step_proc)
        out = set()
        for n in node.nodes:
            for d in get_deps(n, True):
                if d not in produced:
                    out.add(d)
        return set(filter(lambda x: x is not None, out))
    raise TypeError(f"Invalid type in calc_deps: {type(node)}")


def get_res(node, step_proc: bool = False) -> Set[int]:
    """Ids a command produces."""
    from .base import FuseBase
    if isinstance(node, Node):
        proc = node.get_proc() if step_proc else None
        if proc is not None:
            out = []
            for cmd in proc.procedure:
                out.extend(get_res(cmd, True))
            return set(out)
        return set([node.id])
    if isinstance(node, FuseBase):
        out = []
        for n in node.nodes:
            out.extend(get_res(n))
        return set(out)
    raise TypeError(f"Invalid type in calc_res: {type(node)}")


def get_walking_path(node, toposort_res, id_to_node) -> Set[int]:
    """``node`` plus every command in the later layers that (transitively)
    reads it."""
    path = set({node.id})
    for layer in toposort_res:
        for nid in layer:
            n = id_to_node[nid]
            if len(path.intersection(get_deps(n))) > 0:
                path.add(n.id)
    return path
