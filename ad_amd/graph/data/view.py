"""Reshape with the row-major element order unchanged
(autodiff/graph/data/view.py)."""
import math

from ...node import Node

__all__ = ["ViewNode"]


class ViewNode(Node):
    __match_args__ = ("child", "shape")

    def __init__(self, child: Node, shape):
        if math.prod(child.shape) != math.prod(shape):
            raise AssertionError(f"cannot view {child.shape} as {shape}")
        super().__init__([child], shape)

    @staticmethod
    def handle_minus_dim(source_dim, input_dim):
        """``input_dim`` with its -1 (if any) replaced by the size that keeps
        the element count of ``source_dim``."""
        out = list(input_dim)
        if -1 in out:
            known = math.prod(d for d in out if d != -1)
            total = math.prod(source_dim)
            assert total % known == 0, f"{source_dim} has no view as {input_dim}"
            out[out.index(-1)] = total // known
        return out

    def __repr__(self):
        return f"{self.id} = View from {self.children_shapes[0]} to {self.shape} --> ({self.child.id})"

    def repeat_helper(self, is_child):
        return ("View", tuple(self.shape), self.child.repeat_helper(True) if is_child else ())
