"""Graph nodes: identity, operands, listing form, operators and the reverse
pass (the reference's node.py, autodiff/node.py:13-531).

What is fixed by the reference, because every later pass orders its work by
node ids and the listings print them: each node takes the next id when it
is constructed, and each operator constructs its nodes in the same order
as the reference's (``a - b`` builds ``b * -1.0`` before the ``ADD``;
``1 / x`` builds ``x.recip()`` before the constant; ``x.sigmoid()`` is
``1 / (1 + (-x).exp())``; a reverse pass visits a node's left operand's
subtree before its right one).  How that is organised here:

* operators are declared in one table (``_OPERATORS``) of operand builders
  and installed on ``Node``;
* gradient rules live in ``graph/derivatives.py``, one function per node
  kind;
* the reverse pass runs on an explicit work stack (``_ReversePass``).
"""
import math
from copy import deepcopy
from enum import Enum
from typing import List, Optional

from .kernalize import KernelArg, NoneKernelArg


class ChildrenType(Enum):
    SOURCE = 0
    BINARY = 1
    UNARY = 2
    RECEIVER = 3


_CONTEXT_TYPES = []


def _context_types():
    """(Block, Proc), imported on first use (the context module imports this one)."""
    if not _CONTEXT_TYPES:
        from .context import Block, Proc
        _CONTEXT_TYPES.extend((Block, Proc))
    return _CONTEXT_TYPES


class Node:
    """A traced value.  Operands are held as ``child`` (one), ``left`` /
    ``right`` (two) or ``rec_children`` (a Receiver's list); once kernalized,
    ``kargs`` / ``kres`` describe how the kernel reads the operands and
    writes the result."""

    def __init__(self, children, shape: List[int], id_override: Optional[int] = None,
                 is_receiver: bool = False):
        from .context import context
        self.id = context.get_id() if id_override is None else id_override
        for ch in children:
            if not isinstance(ch, Node):
                raise TypeError(f"operand of a graph node must be a node, got {type(ch).__name__}")
        self.children_shapes: List[List[int]] = [deepcopy(ch.shape) for ch in children]
        self.children_datacmds = [[] for _ in children]
        self.kargs: List[KernelArg] = [NoneKernelArg() for _ in children]
        self.kres: KernelArg = NoneKernelArg()
        if not is_receiver:
            for ch in children:
                context.remove_from_dep(ch)        # consumed: no longer a sink of the block
        context.add_to_dep(self)

        self.val = None
        self.incoming_grad = None
        if is_receiver:
            self.children_type = ChildrenType.RECEIVER
            self.rec_children = children            # kept as the caller's list
        elif len(children) == 0:
            self.children_type = ChildrenType.SOURCE
        elif len(children) == 1:
            self.children_type = ChildrenType.UNARY
            (self.child,) = children
        elif len(children) == 2:
            self.children_type = ChildrenType.BINARY
            self.left, self.right = children
        else:
            raise TypeError(f"a graph node takes at most two operands, got {len(children)}")
        self.shape = list(shape)

    # ------------------------------------------------------------------ listing form
    def _label(self) -> str:
        """What the node computes, as the listing prints it (``ADD (6400)``,
        ``Dot Prod [2, 16] x [16, 2]``)."""
        raise NotImplementedError(f"{type(self).__name__} has no listing form")

    def _lowered(self) -> bool:
        return not self.kres.is_none() and not any(k.is_none() for k in self.kargs)

    def __repr__(self) -> str:
        """``<result> = <label> --> (<operands>)``: the kernel operands once
        the node is lowered, operand ids before."""
        if self._lowered():
            operands = ", ".join(str(k) for k in self.kargs)
            return f"{self.kres} = {self._label()} --> ({operands})"
        operands = ", ".join(str(ch.id) for ch in self.children())
        return f"{self.id} = {self._label()} --> ({operands})"

    def repeat_helper(self, is_child=False):
        """Key of the node for merging identical computations (repeat_opt):
        as an operand (``is_child``) or as the operation itself."""
        raise NotImplementedError(f"{type(self).__name__} has no merge key")

    # ------------------------------------------------------------------ structure
    def __hash__(self):
        return hash(self.id)

    def children(self):
        if self.children_type == ChildrenType.RECEIVER:
            return self.rec_children
        if hasattr(self, "left") and hasattr(self, "right"):
            return [self.left, self.right]
        if hasattr(self, "child"):
            return [self.child]
        return []

    def kargs_child_ids(self, filter_temp=False):
        ids = []
        for k in self.kargs:
            ids += k.get_ids(filter_temp)
        return list(set(ids))

    def id_eq(self, other):
        assert isinstance(other, Node), f"cannot compare ids with a {type(other).__name__}"
        return self.id == other.id

    def get_block(self):
        block = getattr(self, "block", None)
        return block if block is not None and isinstance(block, _context_types()[0]) else None

    def get_proc(self):
        proc = getattr(self, "proc", None)
        return proc if proc is not None and isinstance(proc, _context_types()[1]) else None

    def rename(self, fr: int, to: int):
        for k in self.kargs:
            k.rename(fr, to)
        if not self.kres.is_none():
            self.kres.rename(fr, to)
        if self.id == fr:
            self.id = to

    def change_to_temp(self, search: int):
        for k in self.kargs:
            k.change_to_temp(search)
        if not self.kres.is_none():
            self.kres.change_to_temp(search)

    def _to_node(self, value, dim: Optional[List[int]]):
        """A number becomes a constant node of shape ``dim``."""
        from .graph import ConstantNode
        if isinstance(value, (int, float)):
            if dim is None:
                raise TypeError("a number needs a shape to become a node (declare the constant explicitly)")
            return ConstantNode(float(value), dim)
        if not isinstance(value, Node):
            raise TypeError(f"cannot use a {type(value).__name__} as a graph node")
        return value

    # ------------------------------------------------------------------ reverse pass
    def _bck(self, grad):
        from .graph.derivatives import gradient
        return gradient(self, grad)

    def backward(self, grad=None):
        """Propagate ``grad`` (ones of this node's shape when omitted: the
        loss of an implicit ``sum``) back to every node it depends on; a
        node forwards once every consumer has delivered its gradient."""
        _ReversePass(self).run(grad)

    # ------------------------------------------------------------------ unary math
    def exp2(self):
        return self._unary("EXP2")

    def log2(self):
        return self._unary("LOG2")

    def sin(self):
        return self._unary("SIN")

    def sqrt(self):
        return self._unary("SQRT")

    def recip(self):
        return self._unary("RECIP")

    def _unary(self, name):
        from .graph import UnaryNode, UnaryOp
        return UnaryNode(self, UnaryOp[name])

    def cos(self):
        return ((math.pi / 2) - self).sin()

    def exp(self):
        return (self * (1.0 / math.log(2.0))).exp2()

    def ln(self):
        return self.log2() * math.log(2.0)

    def pow2(self):
        return self * self

    def pow3(self):
        return self * self.pow2()

    def powf(self, p: float):
        by_exponent = {2.0: self.pow2, 3.0: self.pow3}
        if p in by_exponent:
            return by_exponent[p]()
        return (p * self.log2()).exp2()

    def sigmoid(self):
        return 1 / (1 + (-self).exp())

    def relu(self):
        return (self > 0) * self

    def softmax(self, dim: int):
        return self.exp() / self.exp().sum(dim).unsqueeze(dim)

    # ------------------------------------------------------------------ shape and data movement
    def broadcast(self, dim: int, size: int):
        from .graph import BroadcastNode
        assert self.shape[dim] == 1, f"only a size-1 axis broadcasts (axis {dim} has {self.shape[dim]})"
        return BroadcastNode(self, dim, size)

    def view(self, target_dim: List[int]):
        from .graph import ViewNode
        target = ViewNode.handle_minus_dim(self.shape, target_dim)
        return self if target == self.shape else ViewNode(self, target)

    def contigious(self):
        from .graph import ContigiousNode
        return ContigiousNode(self)

    def permute(self, order: List[int]):
        from .graph import PermuteNode
        if all(axis == i for i, axis in enumerate(order)):
            return self
        return PermuteNode(self, order)

    def T(self):
        assert len(self.shape) == 2, "T() transposes 2-D nodes"
        return self.permute([1, 0])

    def mT(self):
        assert len(self.shape) == 3, "mT() transposes the last two axes of 3-D nodes"
        return self.permute([0, 2, 1])

    def flatten(self):
        return self.view([math.prod(self.shape)])

    def unsqueeze(self, dim: int):
        at = dim if dim >= 0 else len(self.shape) + dim + 1
        return self.view(self.shape[:at] + [1] + self.shape[at:])

    def squeeze(self, dim: int):
        assert self.shape[dim] == 1, f"squeeze of axis {dim} of size {self.shape[dim]}"
        kept = list(self.shape)
        kept.pop(dim)
        return self.view(kept)

    def __getitem__(self, idx):
        """Slices with step 1 and integer indices, one per leading axis."""
        from .graph import IndexNode
        result, axis = self, 0
        for item in (idx if isinstance(idx, tuple) else (idx,)):
            if isinstance(item, int):
                result = IndexNode(result, item, item + 1, axis).squeeze(axis)
                continue
            if not isinstance(item, slice):
                raise TypeError(f"cannot index a node with a {type(item).__name__}")
            lo = 0 if item.start is None else item.start
            hi = self.shape[axis] if item.stop is None else item.stop
            if hi - lo != self.shape[axis]:
                result = IndexNode(result, lo, hi, axis)
            axis += 1
        return result

    def _reduce_over(self, dim: int, op):
        """Reduce axis ``dim``: swap it last, flatten the rest into rows,
        reduce the rows, restore the leading axes and their order."""
        from .graph import ReduceNode
        rank = len(self.shape)
        axis = dim % rank if dim < 0 else dim
        order = list(range(rank))
        order[axis], order[-1] = order[-1], order[axis]
        moved = self.permute(order)
        kept = list(moved.shape[:-1])
        rows = ReduceNode(moved.view([-1, moved.shape[-1]]), op)
        back = list(order)
        del back[axis]
        return rows.view(kept).permute(back)

    def sum(self, dim: int):
        from .graph import ReduceOp
        return self._reduce_over(dim, ReduceOp.SUM)

    def max(self, dim: int):
        from .graph import ReduceOp
        return self._reduce_over(dim, ReduceOp.MAX)

    def mean(self, dim: int):
        return self.sum(dim) / self.shape[dim]

    def var(self, dim, correction=1):
        centred = (self - self.mean(dim).unsqueeze(dim)).pow2()
        return centred.sum(dim) / (self.shape[dim] - correction)


# ---------------------------------------------------------------------- operators
# Each entry builds ``(left, right, op)`` from ``(self, other)``; operands are
# built left to right, which fixes the order their nodes are created in.
def _c(node, other):
    return node._to_node(other, node.shape)


_OPERATORS = {
    # name: (operand builder, op name, in place)
    "__add__": (lambda s, o: (s, _c(s, o)), "ADD", False),
    "__radd__": (lambda s, o: (s, _c(s, o)), "ADD", False),
    "__mul__": (lambda s, o: (s, _c(s, o)), "MULT", False),
    "__rmul__": (lambda s, o: (s, _c(s, o)), "MULT", False),
    "__sub__": (lambda s, o: (s, _c(s, o) * -1.0), "ADD", False),
    "__rsub__": (lambda s, o: (_c(s, o), s * -1.0), "ADD", False),
    "__truediv__": (lambda s, o: (s, _c(s, o).recip()), "MULT", False),
    "__rtruediv__": (lambda s, o: (s.recip(), _c(s, o)), "MULT", False),
    "__iadd__": (lambda s, o: (s, _c(s, o)), "ADD", True),
    "__isub__": (lambda s, o: (s, _c(s, o) * -1.0), "ADD", True),
    "__itruediv__": (lambda s, o: (s, _c(s, o).recip()), "MULT", True),
    # the reference names its in-place product ``__imult__`` (node.py:306),
    # so ``x *= y`` builds an ordinary product; kept, callable by name
    "__imult__": (lambda s, o: (s, _c(s, o)), "MULT", True),
}

_COMPARISONS = {"__eq__": "EQUAL", "__lt__": "LESS_ZERO", "__le__": "LESS_OR_EQ_ZERO",
                "__gt__": "MORE_ZERO", "__ge__": "MORE_OR_EQ_ZERO"}


def _install_operators(cls):
    def arithmetic(builder, op_name, in_place):
        def method(self, other):
            from .graph import BinaryNode, BinaryOp, try_broadcast
            a, b = try_broadcast(*builder(self, other), only_right_broadcast=in_place)
            return BinaryNode(a, b, BinaryOp[op_name], in_place=in_place)
        return method

    def comparison(op_name):
        def method(self, other):
            from .graph import UnaryNode, UnaryOp
            return UnaryNode(self - other, UnaryOp[op_name])
        return method

    for name, (builder, op_name, in_place) in _OPERATORS.items():
        setattr(cls, name, arithmetic(builder, op_name, in_place))
    for name, op_name in _COMPARISONS.items():
        setattr(cls, name, comparison(op_name))
    cls.__hash__ = lambda self: hash(self.id)      # __eq__ builds a node; hashing stays by id

    def neg(self):
        return self * -1.0

    def matmul(self, other):
        from .graph import DotProdNode
        return DotProdNode(self, self._to_node(other, None))

    def rmatmul(self, other):
        from .graph import DotProdNode
        return DotProdNode(self._to_node(other, None), self)
    cls.__neg__, cls.__matmul__, cls.__rmatmul__ = neg, matmul, rmatmul


_install_operators(Node)


# ---------------------------------------------------------------------- reverse pass
class _ReversePass:
    """Reverse-mode differentiation from a loss node.

    First the consumers of every node reachable from the loss are counted
    (an operand used twice by one node counts twice).  Then gradients are
    delivered from a work stack: a delivery adds to the node's incoming
    gradient (an ``ADD`` node from the second delivery on) and, once every
    consumer has delivered, applies the node's rule and schedules its
    operands' gradients -- the left operand's whole subtree before the right
    one, as a depth-first recursion would."""

    def __init__(self, loss: Node):
        from .context import context
        self.loss = loss
        self.ctx = context

    def _count_consumers(self):
        ctx = self.ctx
        ctx.connections, ctx.grads_seen, ctx.conn_seen = {}, {}, set()
        seen = {self.loss.id}
        stack = [self.loss]
        while stack:
            node = stack.pop()
            for ch in node.children():
                ctx.connections.setdefault(ch.id, []).append(node.id)
                if ch.id not in seen:
                    seen.add(ch.id)
                    stack.append(ch)

    def run(self, grad):
        from .graph import BinaryNode, BinaryOp, ConstantNode
        ctx = self.ctx
        if grad is None:
            self._count_consumers()
            grad = ConstantNode(1.0, self.loss.shape)
        work = [(self.loss, grad)]
        while work:
            node, g = work.pop()
            if node.id in ctx.grads_seen:
                node.incoming_grad = BinaryNode(node.incoming_grad, g, BinaryOp.ADD, False)
                ctx.grads_seen[node.id] += 1
            else:
                node.incoming_grad = g
                ctx.grads_seen[node.id] = 1
            expected = len(ctx.connections.get(node.id, ())) or 1
            if ctx.grads_seen[node.id] != expected:
                continue
            out = node._bck(node.incoming_grad)
            if node.children_type == ChildrenType.UNARY:
                if out is not None:
                    work.append((node.child, out))
            elif node.children_type == ChildrenType.BINARY:
                g_left, g_right = out
                if g_right is not None:
                    work.append((node.right, g_right))
                if g_left is not None:
                    work.append((node.left, g_left))
