"""In-place updates write into their left operand's buffer
(autodiff/opt/in_place.py:7-31): the node's result id becomes the left
operand's id, and every reader is renamed accordingly."""
from ..graph import BinaryNode

__all__ = ["set_in_place"]


def set_in_place(proc):
    repl = {}

    def binary_set(node, _):
        if isinstance(node, BinaryNode) and node.in_place:
            node.kres.rename(node.id, node.left.id)
            repl[node.id] = node.left.id
            node.id = node.left.id
        return node
    proc.walk(binary_set)

    def deps_set(node, _):
        for fr in repl:
            to = repl[fr]
            for idx in range(len(node.kargs)):
                node.kargs[idx].rename(fr, to)
        return node
    proc.walk(deps_set)
    return proc
