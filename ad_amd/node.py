"""Graph node base class: operator overloads and the reverse-mode engine.

Restates autodiff/node.py:13-531.  The order in which every operator creates
its nodes (and therefore requests ids) follows the reference exactly, e.g.
``a - b`` builds ``b * -1.0`` before the ``ADD``; ``1 / x`` builds
``x.recip()`` before the constant.
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


class Node:
    def __init__(self, children, shape: List[int], id_override: Optional[int] = None,
                 is_receiver=False):
        from .context import context

        self.id = context.get_id() if id_override is None else id_override
        self.children_shapes: List[List[int]] = []
        self.children_datacmds = []
        self.kargs: List[KernelArg] = []
        self.kres: KernelArg = NoneKernelArg()
        for ch in children:
            if not isinstance(ch, Node):
                raise TypeError("Children is not type of node!")
            self.children_shapes.append(deepcopy(ch.shape))
            self.children_datacmds.append([])
            self.kargs.append(NoneKernelArg())
            if not is_receiver:
                context.remove_from_dep(ch)
        context.add_to_dep(self)

        self.val = None
        self.children_type = ChildrenType.SOURCE
        if is_receiver:
            self.rec_children = children      # the caller's list, shared on purpose
            self.children_type = ChildrenType.RECEIVER
        elif len(children) == 1:
            self.child = children[0]
            self.children_type = ChildrenType.UNARY
        elif len(children) == 2:
            self.left = children[0]
            self.right = children[1]
            self.children_type = ChildrenType.BINARY
        elif len(children) != 0:
            raise TypeError("Children length is invalid")

        self.incoming_grad = None
        self.shape = list(shape)

    def __repr__(self) -> str:
        raise NotImplementedError

    def repeat_helper(self, is_child=False):
        raise NotImplementedError

    # ------------------------------------------------------------------ autodiff
    def _bck(self, grad):
        raise NotImplementedError

    def _record_connections(self, parent_id=None, visited=None):
        """Count the consumers of every node reachable from the loss
        (node.py:83-105)."""
        from .context import context
        if visited is None:
            visited = set()
        visited.add(self.id)
        if parent_id is not None:
            if self.id not in context.connections:
                context.connections[self.id] = [parent_id]
            else:
                context.connections[self.id].append(parent_id)
        for child in self.children():
            if child.id not in visited:
                child._record_connections(parent_id=self.id, visited=visited)
            else:
                context.connections[child.id].append(self.id)

    def backward(self, grad=None):
        """Accumulate incoming gradients; recurse once all consumers reported
        (node.py:110-152).  With no ``grad`` this is the loss: the seed is a
        ones constant, i.e. an implicit ``sum``."""
        from .context import context
        from .graph import BinaryNode, BinaryOp, ConstantNode

        if grad is None:
            context.grads_seen = dict()
            context.connections = dict()
            context.conn_seen = set()
            self._record_connections(parent_id=None, visited=set())
            grad = ConstantNode(1.0, self.shape)

        if self.id in context.grads_seen:
            self.incoming_grad = BinaryNode(self.incoming_grad, grad, BinaryOp.ADD, False)
            context.grads_seen[self.id] += 1
        else:
            context.grads_seen[self.id] = 1
            self.incoming_grad = grad

        num_connect = len(context.connections[self.id]) if self.id in context.connections else 1
        if num_connect == context.grads_seen[self.id]:
            grad_result = self._bck(self.incoming_grad)
            if self.children_type == ChildrenType.UNARY:
                if grad_result is not None:
                    self.child.backward(grad_result)
            elif self.children_type == ChildrenType.BINARY:
                if grad_result[0] is not None:
                    self.left.backward(grad_result[0])
                if grad_result[1] is not None:
                    self.right.backward(grad_result[1])

    # ------------------------------------------------------------------ helpers
    def __hash__(self):
        return hash(self.id)

    def _to_node(self, node, dim: List[int]):
        from .graph import ConstantNode
        if isinstance(node, int):
            if dim is None:
                raise TypeError("Cannot run dot product on a constant without dim (declare constant manually)")
            return ConstantNode(float(node), dim)
        if isinstance(node, float):
            if dim is None:
                raise TypeError("Cannot run dot product on a constant without dim (declare constant manually)")
            return ConstantNode(node, dim)
        if not isinstance(node, Node):
            raise TypeError(f"Invalid type {type(node)} when converting to node {node}")
        return node

    def children(self):
        from .graph import Receiver
        if isinstance(self, Receiver):
            return self.rec_children
        if hasattr(self, "left") and hasattr(self, "right"):
            return [self.left, self.right]
        if hasattr(self, "child"):
            return [self.child]
        return []

    def kargs_child_ids(self, filter_temp=False):
        ids = []
        for k in self.kargs:
            ids.extend(k.get_ids(filter_temp))
        return list(set(ids))

    def id_eq(self, other):
        assert isinstance(other, Node), "id eq input invalid"
        return self.id == other.id

    def get_block(self):
        if hasattr(self, "block"):
            from .context import Block
            if isinstance(self.block, Block):
                return self.block
        return None

    def get_proc(self):
        if hasattr(self, "proc"):
            from .context import Proc
            if isinstance(self.proc, Proc):
                return self.proc
        return None

    def rename(self, fr: int, to: int):
        for idx in range(len(self.kargs)):
            self.kargs[idx].rename(fr, to)
        if not self.kres.is_none():
            self.kres.rename(fr, to)
        if self.id == fr:
            self.id = to

    def change_to_temp(self, search: int):
        for idx in range(len(self.kargs)):
            self.kargs[idx].change_to_temp(search)
        if not self.kres.is_none():
            self.kres.change_to_temp(search)

    # ------------------------------------------------------------------ binary ops
    def __add__(self, other):
        from .graph import BinaryNode, BinaryOp, try_broadcast
        a, b = try_broadcast(self, self._to_node(other, self.shape))
        return BinaryNode(a, b, BinaryOp.ADD)

    def __radd__(self, other):
        return self.__add__(other)

    def __mul__(self, other):
        from .graph import BinaryNode, BinaryOp, try_broadcast
        a, b = try_broadcast(self, self._to_node(other, self.shape))
        return BinaryNode(a, b, BinaryOp.MULT)

    def __rmul__(self, other):
        return self.__mul__(other)

    def __sub__(self, other):
        from .graph import BinaryNode, BinaryOp, try_broadcast
        a, b = try_broadcast(self, self._to_node(other, self.shape) * -1.0)
        return BinaryNode(a, b, BinaryOp.ADD)

    def __rsub__(self, other):
        from .graph import BinaryNode, BinaryOp, try_broadcast
        a, b = try_broadcast(self._to_node(other, self.shape), self * -1.0)
        return BinaryNode(a, b, BinaryOp.ADD)

    def __truediv__(self, other):
        from .graph import BinaryNode, BinaryOp, try_broadcast
        a, b = try_broadcast(self, self._to_node(other, self.shape).recip())
        return BinaryNode(a, b, BinaryOp.MULT)

    def __rtruediv__(self, other):
        from .graph import BinaryNode, BinaryOp, try_broadcast
        a, b = try_broadcast(self.recip(), self._to_node(other, self.shape))
        return BinaryNode(a, b, BinaryOp.MULT)

    def __neg__(self):
        return self.__mul__(-1.0)

    def __matmul__(self, other):
        from .graph import DotProdNode
        return DotProdNode(self, self._to_node(other, None))

    def __rmatmul__(self, other):
        from .graph import DotProdNode
        return DotProdNode(self._to_node(other, None), self)

    # in-place forms.  ``__imult__`` (not ``__imul__``) is the reference's name
    # (node.py:306), so ``x *= y`` builds an ordinary product there and here.
    def __iadd__(self, other):
        from .graph import BinaryNode, BinaryOp, try_broadcast
        a, b = try_broadcast(self, self._to_node(other, self.shape), only_right_broadcast=True)
        return BinaryNode(a, b, BinaryOp.ADD, in_place=True)

    def __isub__(self, other):
        from .graph import BinaryNode, BinaryOp, try_broadcast
        a, b = try_broadcast(self, self._to_node(other, self.shape) * -1.0, only_right_broadcast=True)
        return BinaryNode(a, b, BinaryOp.ADD, in_place=True)

    def __imult__(self, other):
        from .graph import BinaryNode, BinaryOp, try_broadcast
        a, b = try_broadcast(self, self._to_node(other, self.shape), only_right_broadcast=True)
        return BinaryNode(a, b, BinaryOp.MULT, in_place=True)

    def __itruediv__(self, other):
        from .graph import BinaryNode, BinaryOp, try_broadcast
        a, b = try_broadcast(self, self._to_node(other, self.shape).recip(), only_right_broadcast=True)
        return BinaryNode(a, b, BinaryOp.MULT, in_place=True)

    # ------------------------------------------------------------------ comparisons
    def __eq__(self, other):
        from .graph import UnaryNode, UnaryOp
        return UnaryNode(self - other, UnaryOp.EQUAL)

    def __lt__(self, other):
        from .graph import UnaryNode, UnaryOp
        return UnaryNode(self - other, UnaryOp.LESS_ZERO)

    def __le__(self, other):
        from .graph import UnaryNode, UnaryOp
        return UnaryNode(self - other, UnaryOp.LESS_OR_EQ_ZERO)

    def __gt__(self, other):
        from .graph import UnaryNode, UnaryOp
        return UnaryNode(self - other, UnaryOp.MORE_ZERO)

    def __ge__(self, other):
        from .graph import UnaryNode, UnaryOp
        return UnaryNode(self - other, UnaryOp.MORE_OR_EQ_ZERO)

    # ------------------------------------------------------------------ unary ops
    def _unary(self, op_name):
        from .graph import UnaryNode, UnaryOp
        return UnaryNode(self, UnaryOp[op_name])

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
        if p == 2.0:
            return self.pow2()
        if p == 3.0:
            return self.pow3()
        return (p * self.log2()).exp2()

    # ------------------------------------------------------------------ data movement
    def broadcast(self, dim: int, size: int):
        from .graph import BroadcastNode
        assert self.shape[dim] == 1, "Broadcast dim invalid"
        return BroadcastNode(self, dim, size)

    def view(self, target_dim: List[int]):
        from .graph import ViewNode
        target_dim = ViewNode.handle_minus_dim(self.shape, target_dim)
        if self.shape != target_dim:
            return ViewNode(self, target_dim)
        return self

    def contigious(self):
        from .graph import ContigiousNode
        return ContigiousNode(self)

    def __getitem__(self, idx):
        from .graph import IndexNode
        if not isinstance(idx, tuple):
            idx = (idx,)
        result = self
        dim_counter = 0
        for i in idx:
            if isinstance(i, slice):
                start = 0 if i.start is None else i.start
                sh = self.shape[dim_counter]
                end = sh if i.stop is None else i.stop
                if sh != end - start:
                    result = IndexNode(result, start, end, dim_counter)
                dim_counter += 1
            elif isinstance(i, int):
                result = IndexNode(result, i, i + 1, dim_counter)
                result = result.squeeze(dim_counter)
            else:
                raise TypeError(f"Unsupported index type: {type(i)}")
        return result

    def permute(self, l: List[int]):
        from .graph import PermuteNode
        if sum([l[i] == i for i in range(len(l))]) == len(l):
            return self
        return PermuteNode(self, l)

    def _reduce_proc(self, dim: int, op):
        """Reduce over ``dim`` by permuting it last, viewing 2-D, reducing the
        last axis, then undoing the view and permute (node.py:443-477)."""
        from .graph import ReduceNode
        ndim = len(self.shape)
        if dim < 0:
            dim = ndim + dim
        permute_to = list(range(ndim))
        permute_to[dim], permute_to[-1] = permute_to[-1], permute_to[dim]
        node = self.permute(permute_to)
        new_dim = deepcopy(node.shape)
        last_dim = new_dim[-1]
        node = node.view([-1, last_dim])
        node = ReduceNode(node, op)
        new_dim.pop()
        node = node.view(new_dim)
        permute_back = deepcopy(permute_to)
        del permute_back[dim]
        return node.permute(permute_back)

    def sum(self, dim: int):
        from .graph import ReduceOp
        return Node._reduce_proc(self, dim, ReduceOp.SUM)

    def max(self, dim: int):
        from .graph import ReduceOp
        return Node._reduce_proc(self, dim, ReduceOp.MAX)

    def flatten(self):
        return self.view([math.prod(self.shape)])

    def unsqueeze(self, dim: int):
        if dim < 0:
            dim = len(self.shape) + dim + 1
        d = deepcopy(self.shape)
        d.insert(dim, 1)
        return self.view(d)

    def squeeze(self, dim: int):
        d = deepcopy(self.shape)
        v = d.pop(dim)
        assert v == 1, "Can't squeeze a non-one dim"
        return self.view(d)

    def T(self):
        assert len(self.shape) == 2, "Can't call transpose on a non-2-dim tensor"
        return self.permute([1, 0])

    def mT(self):
        assert len(self.shape) == 3, "Can't call batch transpose on a non-3-dim tensor"
        return self.permute([0, 2, 1])

    def mean(self, dim: int):
        return self.sum(dim) / self.shape[dim]

    def var(self, dim, correction=1):
        a = (self - self.mean(dim).unsqueeze(dim)).pow2()
        return a.sum(dim) / (self.shape[dim] - correction)

    # ------------------------------------------------------------------ nn helpers
    def sigmoid(self):
        return 1 / (1 + (-self).exp())

    def softmax(self, dim: int):
        return self.exp() / self.exp().sum(dim).unsqueeze(dim)

    def relu(self):
        return (self > 0) * self
