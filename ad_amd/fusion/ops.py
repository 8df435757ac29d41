"""The three fused-op families (autodiff/fusion/ops.py:7-50)."""
import math

from ..graph import BinaryNode, DotProdNode, Node, ReduceNode, UnaryNode
from .base import FuseBase

__all__ = ["is_elw", "calc_size", "DPElwFuse", "ReduceElwFuse", "ElwFuse"]


def is_elw(node) -> bool:
    return isinstance(node, UnaryNode) or isinstance(node, BinaryNode)


def calc_size(n):
    if isinstance(n, FuseBase):
        return calc_size(n.nodes[-1])
    if isinstance(n, Node):
        return math.prod(n.shape)


class DPElwFuse(FuseBase):
    """A DotProd followed by elementwise nodes of the same element count."""

    def _fuse(self, node_one, node_two):
        return ((isinstance(node_one, DotProdNode) or is_elw(node_one)) and is_elw(node_two)
                and calc_size(node_one) == calc_size(node_two))

    def _init(self, node):
        return isinstance(node, DotProdNode)


class ReduceElwFuse(FuseBase):
    """A row reduction followed by elementwise nodes over the reduced rows."""

    def _fuse(self, node_one, node_two):
        return ((isinstance(node_one, ReduceNode) or is_elw(node_one)) and is_elw(node_two)
                and calc_size(node_one) == calc_size(node_two))

    def _init(self, node):
        return isinstance(node, ReduceNode)


class ElwFuse(FuseBase):
    """Elementwise nodes of one element count; they need not be connected."""

    def __init__(self):
        super().__init__(dep_match=False)

    def _fuse(self, node_one, node_two):
        return is_elw(node_one) and is_elw(node_two) and calc_size(node_one) == calc_size(node_two)

    def _init(self, node):
        return is_elw(node)
