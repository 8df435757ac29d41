"""SUM or MAX over the last axis of a 2-D operand, [V, R] -> [V]
(autodiff/graph/compute/reduce.py).  Other axes and ranks reach it through
``Node.sum`` / ``Node.max``, which permute and view around it."""
from enum import Enum

from ...node import Node

__all__ = ["ReduceOp", "ReduceNode"]


class ReduceOp(Enum):
    SUM = 1
    MAX = 2


class ReduceNode(Node):
    __match_args__ = ("child", "op")

    def __init__(self, child: Node, op: ReduceOp):
        if len(child.shape) != 2:
            raise AssertionError(f"a reduction takes a 2-D operand, got {child.shape}")
        super().__init__([child], child.shape[:-1])
        self.op = op

    def _label(self):
        rows, length = self.children_shapes[0]
        return f"{self.op.name} on dim: -1 (Vec/X: {rows}, Reduce/Y: {length})"

    def repeat_helper(self, is_child):
        return (self.id,) if is_child else ("Reduce", self.op.value)
