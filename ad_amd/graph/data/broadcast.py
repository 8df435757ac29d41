"""Broadcast along a size-1 axis and the automatic broadcasting rules
(autodiff/graph/data/broadcast.py:6-98)."""
from copy import deepcopy

from ...node import Node

__all__ = ["BroadcastNode", "is_broadcastable", "make_broadcast_node", "try_broadcast"]


class BroadcastNode(Node):
    __match_args__ = ("child", "dim", "size")

    def __init__(self, child: Node, dim: int, size: int):
        p = deepcopy(child.shape)
        p[dim] = size
        super().__init__([child], p)
        self.dim = dim
        self.size = size

    def _bck(self, grad: Node):
        if not isinstance(grad, Node):
            raise TypeError("Grad is not node!")
        return grad.sum(self.dim).unsqueeze(self.dim)

    def __repr__(self) -> str:
        return f"{self.id} = Broadcast dim {self.dim} to size {self.size} --> {self.child.id}"

    def repeat_helper(self, is_child):
        return ("Broadcast", self.dim, self.size,
                self.child.repeat_helper(True) if is_child else ())


def is_broadcastable(dim_a, dim_b) -> bool:
    if not dim_a or not dim_b:
        return False
    for i in range(1, max(len(dim_a), len(dim_b)) + 1):
        a_val = dim_a[-i] if i <= len(dim_a) else 1
        b_val = dim_b[-i] if i <= len(dim_b) else 1
        if a_val != b_val and a_val != 1 and b_val != 1:
            return False
    return True


def make_broadcast_node(n: Node, target_dim) -> Node:
    n_dim = deepcopy(n.shape)
    assert len(target_dim) >= len(n_dim), "Wrong broadcasted node"
    for _ in range(len(target_dim) - len(n_dim)):
        n_dim.insert(0, 1)
    ret = n.view([int(i) for i in n_dim])
    for i in range(len(target_dim)):
        if target_dim[i] != n_dim[i]:
            assert n_dim[i] == 1, f"Can't broadcast node with dim {n_dim} to target dim {target_dim}"
            ret = ret.broadcast(i, target_dim[i])
    return ret


def try_broadcast(a: Node, b: Node, only_right_broadcast: bool = False):
    """Make ``a`` and ``b`` the same shape; constants are left alone (their
    value is shape-free once lowered)."""
    from .constant import ConstantNode
    if len(a.shape) == 0 and len(b.shape) > 0:
        a = a.unsqueeze(0)
    if len(b.shape) == 0 and len(a.shape) > 0:
        b = b.unsqueeze(0)
    if a.shape == b.shape:
        return a, b
    if isinstance(a, ConstantNode) or isinstance(b, ConstantNode):
        return a, b
    if is_broadcastable(a.shape, b.shape):
        if len(a.shape) == len(b.shape):
            broadcast_a = sum(a.shape) < sum(b.shape)
        else:
            broadcast_a = len(a.shape) < len(b.shape)
        if broadcast_a and not only_right_broadcast:
            return make_broadcast_node(a, b.shape), b
        return a, make_broadcast_node(b, a.shape)
    raise ValueError(f"Cannot broadcast {a.shape} to {b.shape}")
