"""Graph-level constant folding (autodiff/opt/simplify.py:12-157).

Rules, first match wins:
  c1 (+|*) c2      -> constant
  (a * c1) * c2    -> a * (c1*c2)     (neither product in place)
  n + 0 / 0 + n    -> n ;  n * 0 / 0 * n -> 0
  n * 1 / 1 * n    -> n
  unary(c)         -> constant (folded in Python float64)
A top-level call re-walks its operands until no rule fires; the "new"
flag is module state shared with nested calls, as in the reference."""
import math

from ..graph import BinaryNode, BinaryOp, ConstantNode, UnaryNode, UnaryOp
from ..helper import walk_graph

__all__ = ["simpl_node"]

is_new = False


def reset_state():
    global is_new
    is_new = False


def _is_const(n, value=None):
    return isinstance(n, ConstantNode) and (value is None or n.constant == value)


_UNARY_FOLD = {
    UnaryOp.EXP2: getattr(math, "exp2", lambda c: 2.0 ** c),   # math.exp2 is 3.11+
    UnaryOp.LOG2: math.log2,
    UnaryOp.SIN: math.sin,
    UnaryOp.RECIP: lambda c: 1.0 / c,
    UnaryOp.SQRT: math.sqrt,
    UnaryOp.EQUAL: lambda c: float(c == 0.0),
    UnaryOp.MORE_ZERO: lambda c: float(c > 0.0),
    UnaryOp.LESS_ZERO: lambda c: float(c < 0.0),
    UnaryOp.MORE_OR_EQ_ZERO: lambda c: float(c >= 0.0),
    UnaryOp.LESS_OR_EQ_ZERO: lambda c: float(c <= 0.0),
}


def _rewrite(node):
    """Return the replacement for ``node`` or None if no rule fires."""
    global is_new
    if isinstance(node, BinaryNode):
        left, right, op = node.left, node.right, node.op
        if _is_const(left) and _is_const(right):
            assert left.shape == right.shape, "shape not equal at simplify constant"
            is_new = True
            val = left.constant + right.constant if op == BinaryOp.ADD else left.constant * right.constant
            return ConstantNode(val, shape=left.shape)
        if (op == BinaryOp.MULT and node.in_place is False and isinstance(left, BinaryNode)
                and left.op == BinaryOp.MULT and left.in_place is False
                and _is_const(left.right) and _is_const(right)):
            assert left.right.shape == right.shape, "shape not equal at simplify constant"
            is_new = True
            return BinaryNode(left.left, ConstantNode(left.right.constant * right.constant,
                                                      shape=left.right.shape),
                              BinaryOp.MULT, False)
        if _is_const(right, 0.0):
            is_new = True
            return left if op == BinaryOp.ADD else ConstantNode(0.0, right.shape)
        if _is_const(left, 0.0):
            is_new = True
            return right if op == BinaryOp.ADD else ConstantNode(0.0, left.shape)
        if op == BinaryOp.MULT and _is_const(right, 1.0):
            is_new = True
            return left
        if op == BinaryOp.MULT and _is_const(left, 1.0):
            is_new = True
            return right
        return None
    if isinstance(node, UnaryNode) and _is_const(node.child):
        is_new = True
        c = node.child.constant
        return ConstantNode(_UNARY_FOLD[node.op](c), node.child.shape)
    return None


def _visit_operands(node, visited):
    if hasattr(node, "left") and hasattr(node, "right"):
        node.left = _inner_simpl(node.left, visited, on_child=True)
        node.right = _inner_simpl(node.right, visited, on_child=True)
        return True
    if hasattr(node, "child"):
        node.child = _inner_simpl(node.child, visited, on_child=True)
        return True
    return False


def _inner_simpl(node, visited, on_child=False):
    global is_new
    if node.id in visited:
        return node
    replacement = _rewrite(node)
    if replacement is not None:
        return replacement
    if not on_child:
        is_new = False
    _visit_operands(node, visited)
    if not on_child:
        while is_new:
            visited = {}
            is_new = False
            if not _visit_operands(node, visited):
                break
    visited[node.id] = 1
    return node


def simpl_node(context):
    context.procedure[0] = walk_graph(context.procedure[0], _inner_simpl,
                                      walk_block=True, walk_child=True)
