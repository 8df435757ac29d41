"""Product of two 2-D operands, [M, K] x [K, N] -> [M, N]
(autodiff/graph/compute/dotprod.py)."""
from ...node import Node

__all__ = ["DotProdNode"]


class DotProdNode(Node):
    __match_args__ = ("left", "right")

    def __init__(self, left: Node, right: Node):
        if len(left.shape) != 2 or len(right.shape) != 2:
            raise AssertionError(f"Dot Prod multiplies 2-D operands, got {left.shape} and {right.shape}")
        if left.shape[1] != right.shape[0]:
            raise AssertionError(f"Dot Prod inner sizes differ: {left.shape} x {right.shape}")
        super().__init__([left, right], shape=[left.shape[0], right.shape[1]])

    def _label(self):
        return f"Dot Prod {self.children_shapes[0]} x {self.children_shapes[1]}"

    def repeat_helper(self, is_child):
        return (self.id,) if is_child else ("DotProd",)
