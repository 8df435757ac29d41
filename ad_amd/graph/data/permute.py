"""Axis permutation (autodiff/graph/data/permute.py:3-39)."""
from ...node import Node

__all__ = ["PermuteNode"]


class PermuteNode(Node):
    __match_args__ = ("child", "permute_to")

    def __init__(self, child: Node, permute_to):
        assert len(child.shape) == len(permute_to), f"permute to invalid dim {len(child.shape)} {permute_to}"
        for i in permute_to:
            assert i < len(child.shape), f"Invalid permute vec: {permute_to} with child shape: {child.shape}"
        dim = [child.shape[permute_to[i]] for i in range(len(child.shape))]
        super().__init__([child], dim)
        self.permute_to = permute_to

    def _bck(self, grad: Node):
        if not isinstance(grad, Node):
            raise TypeError("Grad is not node!")
        inv = [0] * len(self.permute_to)
        for i, p in enumerate(self.permute_to):
            inv[p] = i
        return grad.permute(inv)

    def __repr__(self):
        return f"{self.id} = Permute {self.permute_to} --> {self.child.id}"

    def repeat_helper(self, is_child):
        return ("Permute", tuple(self.permute_to),
                self.child.repeat_helper(True) if is_child else ())
