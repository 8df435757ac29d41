"""Materialise a strided view as a dense buffer
(autodiff/graph/data/contigious.py:7-25)."""
from ...node import Node

__all__ = ["ContigiousNode"]


class ContigiousNode(Node):
    __match_args__ = ("child",)

    def __init__(self, child: Node):
        super().__init__([child], child.shape)

    def _bck(self, grad: Node):
        return grad

    def __repr__(self):
        if self.kargs[0].is_none() or self.kres.is_none():
            return f"{self.id} = Contigious ({self.child.id})"
        return f"{self.kres} = Contigious ({self.child.id}: {self.kargs[0]})"

    def repeat_helper(self, is_child):
        if is_child:
            return (self.id,)
        return ("Contigious",)
