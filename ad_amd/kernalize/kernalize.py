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


def make_karg(initial_dim, child, data_cmds, shape, size_hint: Optional[int] = None, is_concat=False):
    if isinstance(child, ConstantNode):
        return KConstant(child.constant)
    if isinstance(child, ConcatNode):
        dim = ndim_change_datacmds(initial_dim, data_cmds)
        concat_dim = child.dim
        idx_end = child.children_shapes[0][concat_dim]
        dim_two = deepcopy(dim)
        dim_two[concat_dim] = Minus(dim_two[concat_dim], Val(Constant(idx_end)))
        condition = deepcopy(MoreThan(dim[concat_dim], Val(Constant(idx_end - 1))))
        karg_one = make_karg(dim, child.left, child.children_datacmds[0], child.children_shapes[0],
                             is_concat=True)
        karg_two = make_karg(dim_two, child.right, child.children_datacmds[1], child.children_shapes[1],
                             is_concat=True)
        return KConcat(karg_one, karg_two, condition=condition, shape=shape)
    if not is_concat and len(data_cmds) == 0 and initial_dim != [X(), Y()]:
        access = Global()
    else:
        dim = ndim_change_datacmds(initial_dim, data_cmds)
        access = simplify_expr(ndim_to_global(dim, child.shape), size_hint)
    return KMatrix(child.id, access, child.shape)


def make_res_arg(kern_id: int, is_global: bool, shape):
    if is_global:
        return KMatrix(kern_id=kern_id, access=Global(), shape=shape)
    return KMatrix(kern_id=kern_id, access=simplify_expr(ndim_to_global([X(), Y()], shape), None),
                   shape=shape)


def calc_exprs(node, _):
    if isinstance(node, DotProdNode):
        if node.children_datacmds is None:
            return node
        node.kargs[0] = make_karg([X(), Y()], node.left, node.children_datacmds[0], node.children_shapes[0])
        node.kargs[1] = make_karg([X(), Y()], node.right, node.children_datacmds[1], node.children_shapes[1])
        node.kres = make_res_arg(node.id, is_global=False, shape=node.shape)
        node.children_datacmds = None
    elif isinstance(node, BinaryNode):
        if node.children_datacmds is None:
            return node
        size = math.prod(node.shape)
        node.kargs[0] = make_karg(global_to_ndim(Global(), node.children_shapes[0]), node.left,
                                  node.children_datacmds[0], node.children_shapes[0], size_hint=size)
        node.kargs[1] = make_karg(global_to_ndim(Global(), node.children_shapes[1]), node.right,
                                  node.children_datacmds[1], node.children_shapes[1], size_hint=size)
        node.kres = make_res_arg(node.id, is_global=True, shape=node.shape)
        node.children_datacmds = None
    elif isinstance(node, ReduceNode):
        if node.children_datacmds is None:
            return node
        node.kargs[0] = make_karg([X(), Y()], node.child, node.children_datacmds[0], node.children_shapes[0])
        node.kres = make_res_arg(node.id, is_global=False, shape=node.shape)
        node.children_datacmds = None
    elif isinstance(node, (UnaryNode, ContigiousNode)):
        if node.children_datacmds is None:
            return node
        size = math.prod(node.shape)
        node.kargs[0] = make_karg(global_to_ndim(Global(), node.children_shapes[0]), node.child,
                                  node.children_datacmds[0], node.children_shapes[0], size_hint=size)
        node.kres = make_res_arg(node.id, is_global=True, shape=node.shape)
        node.children_datacmds = None
    elif isinstance(node, Feeder):
        node.kres = make_res_arg(node.id, is_global=True, shape=node.shape)
    elif isinstance(node, Receiver):
        if node.children_datacmds is None:
            return node
        ch = node.rec_children
        for idx in range(len(ch)):
            node.kargs[idx] = make_karg(global_to_ndim(Global(), node.children_shapes[idx]), ch[idx],
                                        node.children_datacmds[idx], node.children_shapes[idx],
                                        size_hint=prod(node.children_shapes[idx]))
        node.children_datacmds = None
    return node


def kernalize(context):
    for block in context.procedure:
        for visit in (fill_child_datacmds, calc_exprs):
            block.nodes = walk_graph(block.nodes, visit)
