"""Keep only what has a side effect (autodiff/opt/dep_opt.py:9-57).

A block's top-level nodes are its sinks.  Only loops, Receivers, in-place
updates and Tensor declarations survive; everything else reachable only from
a dropped sink disappears.  A loop whose body ends up empty is removed."""
from ..graph import BinaryNode, Receiver, Tensor
from ..helper import walk_graph
from ..node import Node

__all__ = ["dep_opt"]


def dep_opt(context):
    def filter_node(node, _):
        if not isinstance(node, Node) or node.get_block() is not None:
            return node
        if isinstance(node, Receiver):
            return node
        if isinstance(node, BinaryNode) and node.in_place:
            return node
        if isinstance(node, Tensor):
            return node
        return None

    context.procedure[0] = walk_graph(context.procedure[0], filter_node,
                                      walk_block=True, walk_child=False)
    if len(context.procedure[0].nodes) == 0:
        raise Exception("Empty execution. Make sure to add resultant to dep list")

    def drop_empty_blocks(node):
        block = node.get_block()
        if block is not None:
            if len(block.nodes) == 0:
                return None
            for idx, n in enumerate(block.nodes):
                block.nodes[idx] = drop_empty_blocks(n)
            block.nodes = [n for n in block.nodes if n is not None]
        return node

    main = context.procedure[0]
    for idx, node in enumerate(main.nodes):
        main.nodes[idx] = drop_empty_blocks(node)
    main.nodes = [n for n in main.nodes if n is not None]
