"""Concatenation of two operands along one axis
(autodiff/graph/data/concat.py); ``ad_amd.concat`` chains several."""
from ...node import Node

__all__ = ["ConcatNode"]


class ConcatNode(Node):
    __match_args__ = ("left", "right", "dim")

    def __init__(self, left: Node, right: Node, dim: int):
        if len(left.shape) != len(right.shape):
            raise AssertionError(f"concat of ranks {len(left.shape)} and {len(right.shape)}")
        axis = dim % len(left.shape) if dim < 0 else dim
        others_a = [s for i, s in enumerate(left.shape) if i != axis]
        others_b = [s for i, s in enumerate(right.shape) if i != axis]
        if others_a != others_b:
            raise AssertionError(f"concat along axis {dim} of {left.shape} and {right.shape}")
        shape = list(left.shape)
        shape[dim] += right.shape[dim]
        super().__init__([left, right], shape)
        self.dim = dim

    def __repr__(self):
        return f"{self.id} = Concat at dim: {self.dim} --> ({self.left.id}, {self.right.id})"

    def repeat_helper(self, is_child):
        if is_child:
            return ("Concat", self.dim, self.left.repeat_helper(True), self.right.repeat_helper(True))
        return ("Concat", self.dim, (), ())
