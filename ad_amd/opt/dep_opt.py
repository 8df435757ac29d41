"""Keep only what has a side effect (the behaviour of autodiff/opt/dep_opt.py:9-57).

A block's top-level nodes are its sinks.  Only loops, Receivers, in-place
updates and Tensor declarations survive; everything else reachable only from
a dropped sink disappears.  A loop whose body ends up empty is removed (its
body is checked before the loops inside it are pruned, as the reference
does, so a loop holding only an emptied loop stays)."""
from ..graph import BinaryNode, Receiver, Tensor
from ..helper import walk_graph
from ..node import Node

__all__ = ["dep_opt"]


def _has_effect(node) -> bool:
    """Loops (and anything that is no graph node), Receivers, in-place
    updates and Tensor declarations."""
    if not isinstance(node, Node) or node.get_block() is not None:
        return True
    return isinstance(node, (Receiver, Tensor)) or (isinstance(node, BinaryNode) and node.in_place)


def _without_empty_loops(nodes):
    kept = []
    for node in nodes:
        body = node.get_block()
        if body is not None:
            if not body.nodes:
                continue
            body.nodes = _without_empty_loops(body.nodes)
        kept.append(node)
    return kept


def dep_opt(context):
    main = walk_graph(context.procedure[0], lambda node, _: node if _has_effect(node) else None,
                      walk_block=True, walk_child=False)
    context.procedure[0] = main
    if not main.nodes:
        raise ValueError("nothing to execute: no Receiver, in-place update or loop survives")
    main.nodes = _without_empty_loops(main.nodes)
