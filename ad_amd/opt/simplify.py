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
    _settled.clear()


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


def _operand_names(node):
    if hasattr(node, "left") and hasattr(node, "right"):
        return ("left", "right")
    if hasattr(node, "child"):
        return ("child",)
    return ()


def _visit_operands(node, visited):
    """Simplify the operands in order; (whether ``node`` has operands,
    whether any operand was replaced)."""
    names = _operand_names(node)
    changed = False
    for name in names:
        old = getattr(node, name)
        new = _inner_simpl(old, visited, on_child=True)
        setattr(node, name, new)
        changed |= new is not old
    return bool(names), changed


# ids of nodes already at their fixpoint within the current simpl_node walk:
# no rule fired on the node, none of its operands was replaced while it was
# visited, and every operand is itself in the set.  Nothing beneath such a
# node can change any more, so re-walks skip it (the repeated walk of a
# top-level node's operands after each rewrite was most of the pass's time)
_settled = set()


def _inner_simpl(node, visited, on_child=False):
    global is_new
    if node.id in visited:
        return node
    if node.id in _settled:
        if not on_child:
            is_new = False
        visited[node.id] = 1
        return node
    replacement = _rewrite(node)
    if replacement is not None:
        return replacement
    if not on_child:
        is_new = False
    has_operands, changed = _visit_operands(node, visited)
    if not on_child:
        while is_new:
            visited = {}
            is_new = False
            has_operands, again = _visit_operands(node, visited)
            changed |= again
            if not has_operands:
                break
    visited[node.id] = 1
    if not changed and all(getattr(node, name).id in _settled for name in _operand_names(node)):
        _settled.add(node.id)
    return node


def simpl_node(context):
    _settled.clear()
    context.procedure[0] = walk_graph(context.procedure[0], _inner_simpl,
                                      walk_block=True, walk_child=True)
