"""Structural common-subexpression elimination
(autodiff/opt/repeat_opt.py:12-72).  Two nodes with the same kind and the
same operand ids (data-movement chains compared structurally down to the
source) are merged into the first one found; repeated until nothing merges
(at most 100 rounds)."""
from typing import Any, Dict, List

from ..graph import ConstantNode, Tensor
from ..helper import walk_graph

__all__ = ["repeat_opt"]


def _intern_repeat_opt(context) -> int:
    groups: Dict[Any, List] = {}

    def track_nodes(node, _):
        if node.get_block() is not None:
            return node
        if isinstance(node, Tensor) or isinstance(node, ConstantNode):
            return node
        key = tuple([ch.repeat_helper(is_child=True) for ch in node.children()]) \
            + tuple(node.repeat_helper(is_child=False))
        if key in groups:
            groups[key].append(node)
        else:
            groups[key] = [node]
        return node

    context.procedure[0] = walk_graph(context.procedure[0], track_nodes)
    dupes = [nodes for nodes in groups.values() if len(nodes) > 1]

    # the first group whose later members include the node's id decides
    # (the reference scans the groups in order for every node)
    keep_of = {}
    for nodes in dupes:
        for v in nodes[1:]:
            keep_of.setdefault(v.id, nodes[0])

    def replace_node(node, _):
        return keep_of.get(node.id, node)

    context.procedure[0] = walk_graph(context.procedure[0], replace_node)
    return len(dupes)


def repeat_opt(context):
    merged = 1
    rounds = 0
    while merged > 0:
        merged = _intern_repeat_opt(context)
        rounds += 1
        if rounds >= 100:
            print("Repeat opt max iteration passed")
            break
