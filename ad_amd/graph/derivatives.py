"""Gradient rules, one per node kind: ``gradient(node, grad)`` returns the
gradient of each operand -- a node for one operand, a pair for two, None
where nothing flows back (sources, comparisons).

The rules are the reference's (the ``_bck`` methods of autodiff/graph/) and
build their nodes in the same order: a rule's left-to-right evaluation
creates nodes exactly when the reference's does, so node ids match."""
import math
from copy import deepcopy

from ..node import Node

_RULES = {}


def rule(*kinds):
    def register(fn):
        for k in kinds:
            _RULES[k] = fn
        return fn
    return register


def gradient(node, grad):
    for kind in type(node).__mro__:
        fn = _RULES.get(kind)
        if fn is not None:
            if not isinstance(grad, Node):
                raise TypeError(f"gradient reaching node {node.id} is a {type(grad).__name__}, not a node")
            return fn(node, grad)
    raise TypeError(f"no gradient rule for {type(node).__name__}")


def _install():
    from . import (BinaryNode, BinaryOp, BroadcastNode, ConcatNode, ConstantNode, ContigiousNode, DotProdNode,
                   Feeder, ForNode, IndexNode, PermuteNode, Receiver, ReduceNode, Tensor, UnaryNode, UnaryOp,
                   ViewNode)

    @rule(BinaryNode)
    def _binary(n, g):
        if n.op == BinaryOp.ADD:
            return g, g
        return g * n.right, g * n.left

    per_op = {
        UnaryOp.EXP2: lambda n, g: g * math.log(2.0) * n,
        UnaryOp.LOG2: lambda n, g: g * math.log2(math.e) * n.child.recip(),
        UnaryOp.SIN: lambda n, g: g * n.child.cos(),
        UnaryOp.RECIP: lambda n, g: g * (-1.0 / (n.child.pow2())),
        UnaryOp.SQRT: lambda n, g: g * (1.0 / (2.0 * n.child.sqrt())),
    }

    @rule(UnaryNode)
    def _unary(n, g):
        fn = per_op.get(n.op)
        # comparisons are piecewise constant
        return fn(n, g) if fn is not None else ConstantNode(0.0, n.shape)

    @rule(DotProdNode)
    def _dotprod(n, g):
        return g @ n.right.T(), n.left.T() @ g

    @rule(ReduceNode)
    def _reduce(n, g):
        return g.unsqueeze(-1).broadcast(-1, n.children_shapes[0][-1])

    @rule(BroadcastNode)
    def _broadcast(n, g):
        return g.sum(n.dim).unsqueeze(n.dim)

    @rule(ConcatNode)
    def _concat(n, g):
        cut = n.left.shape[n.dim]
        end = cut + n.right.shape[n.dim]
        return IndexNode(g, 0, cut, n.dim), IndexNode(g, cut, end, n.dim)

    @rule(IndexNode)
    def _index(n, g):
        from .. import concat
        before, after = deepcopy(n.children_shapes[0]), deepcopy(n.children_shapes[0])
        before[n.dim] = n.start
        after[n.dim] = n.children_shapes[0][n.dim] - n.end
        zeros_before = ConstantNode(0, before)
        zeros_after = ConstantNode(0, after)
        return concat([zeros_before, g, zeros_after], n.dim)

    @rule(PermuteNode)
    def _permute(n, g):
        inverse = [0] * len(n.permute_to)
        for position, axis in enumerate(n.permute_to):
            inverse[axis] = position
        return g.permute(inverse)

    @rule(ViewNode)
    def _view(n, g):
        return g.view(n.children_shapes[0])

    @rule(ContigiousNode)
    def _contigious(n, g):
        return g

    @rule(Tensor)
    def _tensor(n, g):
        if n.requires_grad:
            if n.grad_tensor is None:
                n.grad_tensor = g
            else:
                n.grad_tensor += g          # an in-place ADD node
        return None

    @rule(ConstantNode, Feeder, Receiver)
    def _source(n, g):
        return None

    @rule(ForNode)
    def _loop(n, g):
        raise TypeError(f"loop {n.id} has no gradient")


_install()
