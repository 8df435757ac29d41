"""The three fused-op families (autodiff/fusion/ops.py:7-50).

Each family is a first-member kind followed by elementwise nodes (Unary or
Binary) over the same number of elements:

* ``DPElwFuse``     -- a DotProd, then its epilogue;
* ``ReduceElwFuse`` -- a row Reduce, then elementwise work on the reduced
  values;
* ``ElwFuse``       -- elementwise nodes only; members need not read each
  other (independent chains of one size share a kernel).
"""
import math

from ..graph import BinaryNode, DotProdNode, Node, ReduceNode, UnaryNode
from .base import FuseBase

__all__ = ["is_elw", "calc_size", "DPElwFuse", "ReduceElwFuse", "ElwFuse"]


def is_elw(node) -> bool:
    return isinstance(node, (UnaryNode, BinaryNode))


def calc_size(item):
    """Elements a node (or a group's last member) produces."""
    while isinstance(item, FuseBase):
        item = item.nodes[-1]
    if isinstance(item, Node):
        return math.prod(item.shape)
    return None


def _elementwise_after(head_kind):
    """``can_follow`` of a family led by ``head_kind`` (None: any
    elementwise node may lead)."""
    def can_follow(self, member, node):
        leads = is_elw(member) or (head_kind is not None and isinstance(member, head_kind))
        return leads and is_elw(node) and calc_size(member) == calc_size(node)
    return can_follow


class DPElwFuse(FuseBase):
    """A DotProd followed by elementwise nodes of the same element count."""
    can_follow = _elementwise_after(DotProdNode)

    def can_start(self, node):
        return isinstance(node, DotProdNode)


class ReduceElwFuse(FuseBase):
    """A row reduction followed by elementwise nodes over the reduced rows."""
    can_follow = _elementwise_after(ReduceNode)

    def can_start(self, node):
        return isinstance(node, ReduceNode)


class ElwFuse(FuseBase):
    """Elementwise nodes of one element count; they need not be connected."""
    can_follow = _elementwise_after(None)

    def __init__(self):
        super().__init__(dep_match=False)

    def can_start(self, node):
        return is_elw(node)
