"""Broadcasting (autodiff/graph/data/broadcast.py): ``BroadcastNode``
repeats a size-1 axis ``size`` times; ``try_broadcast`` brings the two
operands of an elementwise operation to one shape."""
from ...node import Node

__all__ = ["BroadcastNode", "is_broadcastable", "make_broadcast_node", "try_broadcast"]


class BroadcastNode(Node):
    __match_args__ = ("child", "dim", "size")

    def __init__(self, child: Node, dim: int, size: int):
        shape = list(child.shape)
        shape[dim] = size
        super().__init__([child], shape)
        self.dim = dim
        self.size = size

    def __repr__(self) -> str:
        return f"{self.id} = Broadcast dim {self.dim} to size {self.size} --> {self.child.id}"

    def repeat_helper(self, is_child):
        return ("Broadcast", self.dim, self.size, self.child.repeat_helper(True) if is_child else ())


def is_broadcastable(dim_a, dim_b) -> bool:
    """Trailing-axis rule: aligned from the right, every pair of sizes is
    equal or contains a 1 (missing leading axes count as 1)."""
    if not dim_a or not dim_b:
        return False
    depth = max(len(dim_a), len(dim_b))
    a = [1] * (depth - len(dim_a)) + list(dim_a)
    b = [1] * (depth - len(dim_b)) + list(dim_b)
    return all(x == y or x == 1 or y == 1 for x, y in zip(a, b))


def make_broadcast_node(n: Node, target_dim) -> Node:
    """View ``n`` with leading 1-axes up to the target's rank, then
    broadcast every axis whose size differs, first to last."""
    assert len(target_dim) >= len(n.shape), f"cannot broadcast {n.shape} down to {list(target_dim)}"
    padded = [1] * (len(target_dim) - len(n.shape)) + list(n.shape)
    out = n.view([int(d) for d in padded])
    for axis, (have, want) in enumerate(zip(padded, target_dim)):
        if have != want:
            assert have == 1, f"cannot broadcast {padded} to {list(target_dim)}"
            out = out.broadcast(axis, want)
    return out


def try_broadcast(a: Node, b: Node, only_right_broadcast: bool = False):
    """Operands of an elementwise operation at one shape.  A rank-0 operand
    is viewed as rank 1 first; constants are left as they are (a constant
    has no layout once lowered); otherwise the smaller operand (lower rank,
    or smaller sum of sizes at equal rank) is broadcast to the other, or
    always the right one for an in-place update."""
    from .constant import ConstantNode
    if not a.shape and b.shape:
        a = a.unsqueeze(0)
    if not b.shape and a.shape:
        b = b.unsqueeze(0)
    if a.shape == b.shape or isinstance(a, ConstantNode) or isinstance(b, ConstantNode):
        return a, b
    if not is_broadcastable(a.shape, b.shape):
        raise ValueError(f"shapes {a.shape} and {b.shape} do not broadcast")
    if len(a.shape) == len(b.shape):
        a_smaller = sum(a.shape) < sum(b.shape)
    else:
        a_smaller = len(a.shape) < len(b.shape)
    if a_smaller and not only_right_broadcast:
        return make_broadcast_node(a, b.shape), b
    return a, make_broadcast_node(b, a.shape)
