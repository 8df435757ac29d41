"""Materialise a view chain (permute, view, broadcast, index, concat) as a
dense buffer (autodiff/graph/data/contigious.py)."""
from ...node import Node

__all__ = ["ContigiousNode"]


class ContigiousNode(Node):
    __match_args__ = ("child",)

    def __init__(self, child: Node):
        super().__init__([child], child.shape)

    def __repr__(self):
        if self._lowered():
            return f"{self.kres} = Contigious ({self.child.id}: {self.kargs[0]})"
        return f"{self.id} = Contigious ({self.child.id})"

    def repeat_helper(self, is_child):
        return (self.id,) if is_child else ("Contigious",)
