"""Hoist every remaining non-temp, content-free Alloc to the front of the
main Proc and every non-temp Dealloc to its end
(autodiff/alloc/clean.py:3-28)."""
from . import AllocEntry, DeallocEntry


def temp_clean(proc):
    allocs, deallocs = [], []

    def pick(node, _):
        if isinstance(node, AllocEntry):
            if node.is_temp or node.content is not None:
                return node
            allocs.append(node)
        elif isinstance(node, DeallocEntry):
            if not node.is_temp:
                deallocs.append(node)
            else:
                return None
        else:
            return node
        return None
    proc.walk(pick)
    for a in allocs:
        proc.insert(0, a)
    for d in deallocs:
        proc.append(d)
