"""Index algebra of data-movement chains, and the graph walk the compile
passes use to visit or replace nodes (the behaviour of autodiff/helper.py:19-135).

The access expressions built here are printed in the Proc listing and
compared with the reference's text, so each function builds the same tree
the reference does: strides as ``Val(Constant(int))``, a flat index split
as ``(index / stride) % extent`` with one shared ``index`` object, and a
flat index joined as the left-nested sum of ``dim_i * stride_i``.
"""
from copy import deepcopy
from typing import Callable, List

from .context import Block, indent_str  # noqa: F401  (indent_str re-exported)
from .expr import Add, Constant, Div, Minus, Mult, Remainder, Val
from .node import Node


def _const(v: int):
    return Val(Constant(v))


def _row_major(shape: List[int]) -> List[int]:
    """Integer strides of a row-major ``shape`` (last axis 1)."""
    out, step = [], 1
    for extent in reversed(shape):
        out.append(step)
        step *= extent
    out.reverse()
    return out


def calc_stride(shape: List[int]):
    """Row-major strides as constant expressions."""
    return [_const(s) for s in _row_major(shape)]


def global_to_ndim(index, shape: List[int]):
    """Per-axis coordinates of a flat ``index``: ``(index / stride) % extent``."""
    return [Remainder(Div(index, stride), _const(extent))
            for stride, extent in zip(calc_stride(shape), shape)]


def ndim_to_global(dim, shape: List[int]):
    """Flat index of per-axis coordinates, summed from the first axis on."""
    terms = [Mult(d, s) for d, s in zip(dim, calc_stride(shape))]
    total = terms[0]
    for t in terms[1:]:
        total = Add(total, t)
    return total


# --- coordinates seen through one data-movement node ------------------------
# Each rule maps the coordinates a consumer uses to those of the node's
# input (helper.py:52-73); Broadcast and Index edit the list they are given.

def _through_permute(node, dim):
    return [deepcopy(dim[src]) for src in node.permute_to]


def _through_view(node, dim):
    return global_to_ndim(ndim_to_global(dim, node.shape), node.children_shapes[0])


def _through_broadcast(node, dim):
    dim[node.dim] = _const(0)
    return dim


def _through_index(node, dim):
    axis, start = node.dim, node.start
    # a negative start is the offset of a concat piece (concat -> index)
    dim[axis] = Minus(dim[axis], _const(-start)) if start < 0 else Add(dim[axis], _const(start))
    return dim


def _coordinate_rules():
    from .graph import BroadcastNode, IndexNode, PermuteNode, ViewNode
    return ((PermuteNode, _through_permute), (ViewNode, _through_view),
            (BroadcastNode, _through_broadcast), (IndexNode, _through_index))


def ndim_change_datacmds(dim, data_cmds: List[Node]):
    """Coordinates of the source of a chain of data-movement nodes, given
    those the consumer at the end of the chain uses."""
    rules = _coordinate_rules()
    for cmd in data_cmds:
        for kind, rule in rules:
            if isinstance(cmd, kind):
                dim = rule(cmd, dim)
                break
    return dim


# --- the graph walk ----------------------------------------------------------
# ids of the nodes handed to the visitor during the current walk; visitors
# receive this dict and may consult or fill it (context.reset clears it)
visited = {}


def _operand_slots(node):
    """(read, write) accessors of the operands the walk descends into, in
    order: a Receiver's list, else ``child``, else ``left`` then ``right``.
    Each read happens when its slot is reached, after the earlier slots'
    subtrees were walked."""
    from .graph import Receiver
    if isinstance(node, Receiver):
        kids = node.rec_children
        return [(lambda i=i: kids[i], lambda v, i=i: kids.__setitem__(i, v))
                for i in range(len(kids))]
    names = ("child",) if hasattr(node, "child") else \
        ("left", "right") if (hasattr(node, "left") and hasattr(node, "right")) else ()
    return [(lambda a=a: getattr(node, a), lambda v, a=a: setattr(node, a, v)) for a in names]


def _visit(node: Node, f: Callable, into_blocks: bool, into_operands: bool, kwargs):
    """Hand ``node`` to ``f``; walk what its replacement holds.  A result of
    ``None`` removes the node from the list or block that holds it."""
    out = f(node, visited, **kwargs)
    visited[node.id] = 1
    if out is None:
        return None
    body = out.get_block()
    if body is not None:
        if into_blocks:
            walked = walk_graph(body.nodes, f, into_blocks, into_operands, reset_visited=False, **kwargs)
            out.block.nodes = [x for x in walked if x is not None]
        return out
    if into_operands:
        for read, write in _operand_slots(out):
            operand = read()
            if operand.id not in visited:
                write(_visit(operand, f, into_blocks, into_operands, kwargs))
    return out


def walk_graph(n, f: Callable, walk_block=True, walk_child=True, reset_visited=True, **kwargs):
    """Depth-first walk calling ``f(node, visited, **kwargs)`` on a Block, a
    non-empty list of nodes or one node.  ``f`` returns the node to keep (a
    replacement is walked in its place) or ``None`` to drop it from the
    enclosing list.  Every entry of a list is handed to ``f``; an operand
    only once per walk.  Loop bodies are walked when ``walk_block``,
    operands when ``walk_child``."""
    if reset_visited:
        visited.clear()
    if isinstance(n, Block):
        n.nodes = walk_graph(n.nodes, f, walk_block, walk_child, **kwargs)
        return n
    if isinstance(n, list) and n and isinstance(n[0], Node):
        kept = (_visit(x, f, walk_block, walk_child, kwargs) for x in n)
        return [x for x in kept if x is not None]
    if isinstance(n, Node):
        return _visit(n, f, walk_block, walk_child, kwargs)
    raise TypeError(f"Invalid type {type(n)} in walk_graph")
