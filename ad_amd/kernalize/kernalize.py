"""Fold data-movement chains into per-operand access expressions
(autodiff/kernalize/kernalize.py:19-254).

Conventions: DotProd and Reduce operands and results are addressed with
``X``/``Y`` (row, column); elementwise operands with ``Global`` decomposed by
the operand's strides; a Feeder's result is ``Global``; Receiver operands
must be contiguous."""
import math
from copy import deepcopy
from math import prod
from typing import Optional

from ..expr import Constant, Global, Minus, MoreThan, Val, X, Y
from ..expr.simplify import simplify_expr
from ..graph import (BinaryNode, BroadcastNode, ConcatNode, ConstantNode, ContigiousNode,
                     DotProdNode, Feeder, IndexNode, PermuteNode, Receiver, ReduceNode,
                     UnaryNode, ViewNode)
from ..helper import global_to_ndim, ndim_change_datacmds, ndim_to_global, walk_graph
from . import KConcat, KConstant, KMatrix

_DATA_CMDS = (PermuteNode, ViewNode, BroadcastNode, IndexNode)


def pot_child_datacmd(node, mandate_contigious=False):
    """(source, peeled data cmd or None, peeled?)"""
    if len(node.children()) == 0:
        return (node, None, False)
    if isinstance(node, _DATA_CMDS):
        if mandate_contigious:
            raise Exception("A non contigious node is found where suppose to be contigious")
        return (node.child, node, True)
    return (node, None, False)


def _peel(get, put, sink, mandate=False):
    while True:
        src, cmd, did = pot_child_datacmd(get(), mandate)
        put(src)
        if cmd is not None:
            sink.append(cmd)
        if not did:
            break


def fill_child_datacmds(node, _):
    """Strip data-movement nodes off every operand, remembering them in
    ``children_datacmds`` (outermost first)."""
    if isinstance(node, (DotProdNode, BinaryNode, ConcatNode)):
        _peel(lambda: node.left, lambda v: setattr(node, "left", v), node.children_datacmds[0])
        _peel(lambda: node.right, lambda v: setattr(node, "right", v), node.children_datacmds[1])
    elif isinstance(node, (ReduceNode, UnaryNode, ContigiousNode)):
        _peel(lambda: node.child, lambda v: setattr(node, "child", v), node.children_datacmds[0])
    elif isinstance(node, Receiver):
        for idx in range(len(node.rec_children)):
            _peel(lambda: node.rec_children[idx],
                  lambda v: node.rec_children.__setitem__(idx, v),
                  node.children_datacmds[idx], mandate=True)
    return node


def _matrix_operand(coords, node, data_cmds, size_hint, in_concat):
    """A buffer read: ``Global`` when an elementwise read goes straight to
    the buffer, else the flat index of the source coordinates the chain of
    data-movement nodes maps ``coords`` to."""
    if not in_concat and len(data_cmds) == 0 and coords != [X(), Y()]:
        return KMatrix(node.id, Global(), node.shape)
    source = ndim_change_datacmds(coords, data_cmds)
    return KMatrix(node.id, simplify_expr(ndim_to_global(source, node.shape), size_hint), node.shape)


def _concat_operand(coords, node, data_cmds, shape):
    """A concat read as a selection between its two pieces: the second
    where the coordinate along the concat axis is past the first piece
    (shifted back by the first piece's extent), else the first."""
    coords = ndim_change_datacmds(coords, data_cmds)
    axis = node.dim
    split = node.children_shapes[0][axis]
    # fixed before the first piece is built: building a piece may edit the
    # coordinate list it is given
    second = deepcopy(coords)
    second[axis] = Minus(second[axis], Val(Constant(split)))
    selects_second = deepcopy(MoreThan(coords[axis], Val(Constant(split - 1))))
    pieces = [make_karg(coords, node.left, node.children_datacmds[0], node.children_shapes[0], is_concat=True)]
    pieces.append(make_karg(second, node.right, node.children_datacmds[1], node.children_shapes[1],
                            is_concat=True))
    return KConcat(pieces[0], pieces[1], condition=selects_second, shape=shape)


def make_karg(initial_dim, child, data_cmds, shape, size_hint: Optional[int] = None, is_concat=False):
    """Kernel operand that reads ``child`` (through the data-movement nodes
    ``data_cmds``) at the coordinates ``initial_dim`` of the consumer."""
    if isinstance(child, ConstantNode):
        return KConstant(child.constant)
    if isinstance(child, ConcatNode):
        return _concat_operand(initial_dim, child, data_cmds, shape)
    return _matrix_operand(initial_dim, child, data_cmds, size_hint, is_concat)


def make_res_arg(kern_id: int, is_global: bool, shape):
    """The result of a node: its flat index, or (row, column) of a tile."""
    access = Global() if is_global else simplify_expr(ndim_to_global([X(), Y()], shape), None)
    return KMatrix(kern_id=kern_id, access=access, shape=shape)


# how a node's operands are read: at the (row, column) of a DotProd or
# Reduce tile, or at the coordinates of the consumer's flat index
_TILE, _FLAT = "tile", "flat"


def _reads(node):
    """(operands, index space, size hint per operand, result written by
    flat index / by tile / not at all) of a node whose operands become
    kernel args, else None."""
    if isinstance(node, DotProdNode):
        return [node.left, node.right], _TILE, [None, None], _TILE
    if isinstance(node, BinaryNode):
        n = math.prod(node.shape)
        return [node.left, node.right], _FLAT, [n, n], _FLAT
    if isinstance(node, ReduceNode):
        return [node.child], _TILE, [None], _TILE
    if isinstance(node, (UnaryNode, ContigiousNode)):
        return [node.child], _FLAT, [math.prod(node.shape)], _FLAT
    if isinstance(node, Receiver):
        return list(node.rec_children), _FLAT, [prod(s) for s in node.children_shapes], None
    return None


def calc_exprs(node, _):
    """Replace ``node``'s operands and result by kernel args (once: the data
    command lists are dropped afterwards)."""
    if isinstance(node, Feeder):
        node.kres = make_res_arg(node.id, is_global=True, shape=node.shape)
        return node
    layout = _reads(node)
    if layout is None or node.children_datacmds is None:
        return node
    operands, space, hints, result = layout
    for i, (child, hint) in enumerate(zip(operands, hints)):
        shape = node.children_shapes[i]
        coords = [X(), Y()] if space == _TILE else global_to_ndim(Global(), shape)
        node.kargs[i] = make_karg(coords, child, node.children_datacmds[i], shape, size_hint=hint)
    if result is not None:
        node.kres = make_res_arg(node.id, is_global=result == _FLAT, shape=node.shape)
    node.children_datacmds = None
    return node


def kernalize(context):
    for block in context.procedure:
        for visit in (fill_child_datacmds, calc_exprs):
            block.nodes = walk_graph(block.nodes, visit)
