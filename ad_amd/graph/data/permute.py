"""Axis permutation: axis i of the result is axis ``permute_to[i]`` of the
operand (autodiff/graph/data/permute.py)."""
from ...node import Node

__all__ = ["PermuteNode"]


class PermuteNode(Node):
    __match_args__ = ("child", "permute_to")

    def __init__(self, child: Node, permute_to):
        rank = len(child.shape)
        if len(permute_to) != rank or any(axis >= rank for axis in permute_to):
            raise AssertionError(f"{permute_to} does not permute the axes of {child.shape}")
        super().__init__([child], [child.shape[axis] for axis in permute_to])
        self.permute_to = permute_to

    def __repr__(self):
        return f"{self.id} = Permute {self.permute_to} --> {self.child.id}"

    def repeat_helper(self, is_child):
        return ("Permute", tuple(self.permute_to), self.child.repeat_helper(True) if is_child else ())
