"""Row reduction over the last axis of a 2-D operand
(autodiff/graph/compute/reduce.py:6-43)."""
from copy import deepcopy
from enum import Enum

from ...node import Node

__all__ = ["ReduceOp", "ReduceNode"]


class ReduceOp(Enum):
    SUM = 1
    MAX = 2


class ReduceNode(Node):
    __match_args__ = ("child", "op")

    def __init__(self, child: Node, op: ReduceOp):
        assert len(child.shape) == 2, "Reduce shape must be 2-dim"
        res_shape = deepcopy(child.shape)
        del res_shape[-1]
        super().__init__([child], res_shape)
        self.op = op

    def _bck(self, grad: Node):
        repeat_n = self.children_shapes[0][-1]
        return grad.unsqueeze(-1).broadcast(-1, repeat_n)

    def __repr__(self):
        sh = self.children_shapes[0]
        size_str = f"(Vec/X: {sh[0]}, Reduce/Y: {sh[1]})"
        if self.kargs[0].is_none() or self.kres.is_none():
            return f"{self.id} = {self.op.name} on dim: -1 {size_str} --> ({self.child.id})"
        return f"{self.kres} = {self.op.name} on dim: -1 {size_str} --> ({self.kargs[0]})"

    def repeat_helper(self, is_child):
        if is_child:
            return (self.id,)
        return ("Reduce", self.op.value)
