"""Stride/index math and the graph walker (autodiff/helper.py:19-135)."""
from copy import deepcopy
from typing import Callable, List

from .context import Block, indent_str  # noqa: F401  (indent_str re-exported)
from .expr import Add, Constant, Div, Minus, Mult, Remainder, Val
from .node import Node


def calc_stride(shape: List[int]):
    """Row-major strides as constant expressions."""
    n = len(shape)
    strides = [Val(Constant(1)) for _ in range(n)]
    for i in reversed(range(n - 1)):
        strides[i] = Val(Constant(strides[i + 1].get_const() * shape[i + 1]))
    return strides


def global_to_ndim(index, shape: List[int]):
    """``[(index / stride_i) % shape_i]``; every component shares ``index``."""
    strides = calc_stride(shape)
    return [Remainder(Div(index, strides[i]), Val(Constant(shape[i]))) for i in range(len(shape))]


def ndim_to_global(dim, shape: List[int]):
    """``sum_i dim_i * stride_i`` built left to right."""
    strides = calc_stride(shape)
    expr = Mult(dim[0], strides[0])
    for i in range(1, len(shape)):
        expr = Add(expr, Mult(dim[i], strides[i]))
    return expr


def ndim_change_datacmds(dim, data_cmds: List[Node]):
    """Map per-axis index expressions of a consumer back through a chain of
    data-movement nodes to the coordinates of their source
    (helper.py:52-73).  Broadcast and Index edit ``dim`` in place."""
    from .graph import BroadcastNode, IndexNode, PermuteNode, ViewNode
    for cmd in data_cmds:
        if isinstance(cmd, PermuteNode):
            perm = cmd.permute_to
            new_dim = [Val(Constant(0)) for _ in range(len(dim))]
            for i in range(len(dim)):
                new_dim[i] = deepcopy(dim[perm[i]])
            dim = new_dim
        elif isinstance(cmd, ViewNode):
            dim = global_to_ndim(ndim_to_global(dim, cmd.shape), cmd.children_shapes[0])
        elif isinstance(cmd, BroadcastNode):
            dim[cmd.dim] = Val(Constant(0))
        elif isinstance(cmd, IndexNode):
            d, start = cmd.dim, cmd.start
            if start < 0:
                dim[d] = Minus(dim[d], Val(Constant(abs(start))))
            else:
                dim[d] = Add(dim[d], Val(Constant(start)))
    return dim


# ids already handed to ``f`` during the current walk (helper.py:76)
visited = {}


def _walk_node(n: Node, f: Callable, walk_block=True, walk_child=True, **kwargs):
    res = f(n, visited, **kwargs)
    visited[n.id] = 1
    if res is None:
        return None
    block = res.get_block()
    if block is not None:
        if walk_block:
            block_nodes = walk_graph(block.nodes, f, walk_block, walk_child, reset_visited=False, **kwargs)
            res.block.nodes = [x for x in block_nodes if x is not None]
    elif walk_child:
        from .graph import Receiver
        if isinstance(res, Receiver):
            for idx in range(len(res.rec_children)):
                ch = res.rec_children[idx]
                if ch.id not in visited:
                    res.rec_children[idx] = _walk_node(ch, f, walk_block, walk_child, **kwargs)
        elif hasattr(res, "child"):
            if res.child.id not in visited:
                res.child = _walk_node(res.child, f, walk_block, walk_child, **kwargs)
        elif hasattr(res, "left") and hasattr(res, "right"):
            if res.left.id not in visited:
                res.left = _walk_node(res.left, f, walk_block, walk_child, **kwargs)
            if res.right.id not in visited:
                res.right = _walk_node(res.right, f, walk_block, walk_child, **kwargs)
    return res


def walk_graph(n, f: Callable, walk_block=True, walk_child=True, reset_visited=True, **kwargs):
    """Depth-first walk calling ``f(node, visited)``; ``f`` may return a
    replacement node or ``None`` to drop it (helper.py:111-135).  Top-level
    list entries are always visited; children only once per walk."""
    if reset_visited:
        visited.clear()
    if isinstance(n, Block):
        n.nodes = walk_graph(n.nodes, f, walk_block, walk_child, **kwargs)
        return n
    if isinstance(n, list) and len(n) > 0 and isinstance(n[0], Node):
        out = []
        for node in n:
            res = _walk_node(node, f, walk_block, walk_child, **kwargs)
            if res is not None:
                out.append(res)
        return out
    if isinstance(n, Node):
        return _walk_node(n, f, walk_block, walk_child, **kwargs)
    raise TypeError(f"Invalid type {type(n)} in walk_graph")
