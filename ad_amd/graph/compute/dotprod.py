"""2-D matrix product (autodiff/graph/compute/dotprod.py:5-39)."""
from ...node import Node

__all__ = ["DotProdNode"]


class DotProdNode(Node):
    __match_args__ = ("left", "right")

    def __init__(self, left: Node, right: Node):
        assert len(left.shape) == 2, "Left shape of dot prod must be 2"
        assert len(right.shape) == 2, "Right shape of dot prod must be 2"
        assert left.shape[1] == right.shape[0], \
            f"Dot product dim mismatch. left: {left.shape} right: {right.shape}"
        super().__init__([left, right], shape=[left.shape[0], right.shape[1]])

    def _bck(self, grad: Node):
        return grad @ self.right.T(), self.left.T() @ grad

    def __repr__(self):
        size_str = f"{self.children_shapes[0]} x {self.children_shapes[1]}"
        if self.kargs[0].is_none() or self.kargs[1].is_none() or self.kres.is_none():
            return f"{self.id} = Dot Prod {size_str} --> ({self.left.id}, {self.right.id})"
        return f"{self.kres} = Dot Prod {size_str} --> ({self.kargs[0]}, {self.kargs[1]})"

    def repeat_helper(self, is_child):
        if is_child:
            return (self.id,)
        return ("DotProd",)
