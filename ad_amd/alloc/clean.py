"""Hoist every remaining non-temp, content-free Alloc to the front of the
main Proc and every non-temp Dealloc to its end; temp Deallocs are dropped
(the behaviour of autodiff/alloc/clean.py:3-28)."""
from . import AllocEntry, DeallocEntry


def temp_clean(proc):
    allocs, deallocs = [], []

    def sift(node, _):
        if isinstance(node, DeallocEntry):
            if not node.is_temp:
                deallocs.append(node)
            return None                      # a temp's free is implicit (registers)
        if isinstance(node, AllocEntry) and not node.is_temp and node.content is None:
            allocs.append(node)
            return None
        return node
    proc.walk(sift)
    # each collected Alloc goes to the front in turn: the last one first
    proc.procedure[:0] = allocs[::-1]
    proc.procedure.extend(deallocs)
