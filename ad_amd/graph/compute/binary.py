"""Elementwise sum and product of two same-shape operands
(autodiff/graph/compute/binary.py).  ``in_place`` marks an update written
into the left operand's buffer (the SGD step)."""
import math
from enum import Enum

from ...node import Node

__all__ = ["BinaryOp", "BinaryNode"]


class BinaryOp(Enum):
    ADD = 1
    MULT = 2


class BinaryNode(Node):
    __match_args__ = ("left", "right", "op", "in_place")

    def __init__(self, left: Node, right: Node, op: BinaryOp, in_place: bool = False):
        if left.shape != right.shape:
            raise AssertionError(f"{op.name} of shapes {left.shape} ({left}) and {right.shape} ({right})")
        super().__init__([left, right], left.shape, None)
        self.op = op
        self.in_place = in_place

    def _label(self):
        mode = " IN PLACE" if self.in_place else ""
        return f"{self.op.name}{mode} ({math.prod(self.shape)})"

    def repeat_helper(self, is_child):
        return (self.id,) if is_child else ("Binary", self.op.value, self.in_place)
