"""Reshape without moving data (autodiff/graph/data/view.py:5-47)."""
import math

from ...node import Node

__all__ = ["ViewNode"]


class ViewNode(Node):
    __match_args__ = ("child", "shape")

    def __init__(self, child: Node, shape):
        assert math.prod(child.shape) == math.prod(shape), "View dimensions are incorrect"
        super().__init__([child], shape)

    @staticmethod
    def handle_minus_dim(source_dim, input_dim):
        if -1 in input_dim:
            idx = input_dim.index(-1)
            total = math.prod(source_dim)
            known = math.prod(d for d in input_dim if d != -1)
            assert total % known == 0, "Can't fill in -1"
            input_dim = input_dim.copy()
            input_dim[idx] = total // known
        return list(input_dim)

    def _bck(self, grad: Node):
        if not isinstance(grad, Node):
            raise TypeError("Grad is not node!")
        return grad.view(self.children_shapes[0])

    def __repr__(self):
        return f"{self.id} = View from {self.children_shapes[0]} to {self.shape} --> ({self.child.id})"

    def repeat_helper(self, is_child):
        return ("View", tuple(self.shape),
                self.child.repeat_helper(True) if is_child else ())
