"""Structural common-subexpression elimination (the behaviour of
autodiff/opt/repeat_opt.py:12-72).

Two nodes are interchangeable when their merge keys are equal: the node's
own ``repeat_helper`` (kind and parameters) after those of its operands
(a data-movement chain is compared by structure down to its source).  In a
round, every node is noted under its key in walk order, and every later
member of a key is replaced by the first; rounds repeat until one merges
nothing (at most 100)."""
from typing import Any, Dict, List

from ..graph import ConstantNode, Tensor
from ..helper import walk_graph

__all__ = ["repeat_opt"]

_MAX_ROUNDS = 100


def _mergeable(node) -> bool:
    """Loops, Tensors and constants are never merged."""
    return node.get_block() is None and not isinstance(node, (Tensor, ConstantNode))


def _merge_key(node):
    return tuple(operand.repeat_helper(is_child=True) for operand in node.children()) \
        + tuple(node.repeat_helper(is_child=False))


def _one_round(context) -> int:
    """One round; returns the number of keys noted more than once (a node
    noted twice under its key counts, as in the reference)."""
    noted: Dict[Any, List] = {}

    def note(node, _):
        if _mergeable(node):
            noted.setdefault(_merge_key(node), []).append(node)
        return node
    context.procedure[0] = walk_graph(context.procedure[0], note)

    survivor = {}
    repeated = 0
    for members in noted.values():
        if len(members) > 1:
            repeated += 1
            for later in members[1:]:
                survivor.setdefault(later.id, members[0])
    context.procedure[0] = walk_graph(context.procedure[0], lambda node, _: survivor.get(node.id, node))
    return repeated


def repeat_opt(context):
    for rounds in range(1, _MAX_ROUNDS + 1):
        repeated = _one_round(context)
        if rounds == _MAX_ROUNDS:
            print("Repeat opt max iteration passed")
            return
        if repeated == 0:
            return
