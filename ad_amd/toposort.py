"""Kahn layering with the exact set/dict construction order of the
``toposort`` package (1.x, ``toposort(data)``), which the reference imports
at autodiff/linearize.py:10 and autodiff/fusion/helper.py:6 without a pinned
version.

The layer *contents* are fixed by the algorithm; the iteration order inside
each layer is CPython set order, which depends on how each set was built.
The reference's command order (and so its arena offsets) comes from that
iteration order, so this module performs the same container operations in
the same sequence: drop self-edges in place, add every dependency that is
not a key as a key with no dependencies, then repeatedly emit the set of keys
whose dependency set is empty and subtract it from the rest.
"""
from functools import reduce


class CircularDependencyError(ValueError):
    def __init__(self, data):
        super().__init__(f"Circular dependencies exist among these items: {data!r}")
        self.data = data


def toposort(data):
    if len(data) == 0:
        return
    data = data.copy()
    for item, deps in data.items():
        deps.discard(item)
    extra = reduce(set.union, data.values()) - set(data.keys())
    data.update({item: set() for item in extra})
    while True:
        ordered = set(item for item, dep in data.items() if len(dep) == 0)
        if not ordered:
            break
        yield ordered
        data = {item: (dep - ordered) for item, dep in data.items() if item not in ordered}
    if len(data) != 0:
        raise CircularDependencyError(data)
