"""In-place updates (autodiff/opt/in_place.py:7-31).

An in-place ``BinaryNode`` (``x += g``, the SGD update) must write into the
buffer of its left operand instead of a buffer of its own.  Its result slot
and its id are moved to the left operand's id; then every operand anywhere
in the Proc that read the node's old id reads the left operand's id.  The
rename table is applied to each operand in the order its entries were
made, which matters when an update's target is itself an earlier update."""
from ..graph import BinaryNode

__all__ = ["set_in_place"]


def set_in_place(proc):
    moved = {}                     # old result id -> id of the updated buffer

    def redirect_result(node, _):
        if isinstance(node, BinaryNode) and node.in_place:
            target = node.left.id
            node.kres.rename(node.id, target)
            moved[node.id] = target
            node.id = target
        return node

    def redirect_reads(node, _):
        for old, new in moved.items():
            for karg in node.kargs:
                karg.rename(old, new)
        return node

    proc.walk(redirect_result)
    proc.walk(redirect_reads)
    return proc
