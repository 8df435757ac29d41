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
    """Yield the Kahn layers of ``data`` (item -> set of items it depends on).

    Each yielded set is built by inserting its items in the key order of the
    working dict, exactly as ``set(item for item, dep in data.items() if
    len(dep) == 0)`` does in the package, so its iteration order matches.
    The package recomputes every remaining dependency set once per layer;
    here each item's layer is found with one pass of in-degree counting,
    which gives the same layers in O(items + edges)."""
    if len(data) == 0:
        return
    data = data.copy()
    for item, deps in data.items():
        deps.discard(item)
    extra = reduce(set.union, data.values()) - set(data.keys())
    data.update({item: set() for item in extra})

    position = {item: i for i, item in enumerate(data)}
    remaining = {item: len(deps) for item, deps in data.items()}
    dependents = {}
    for item, deps in data.items():
        for d in deps:
            dependents.setdefault(d, []).append(item)
    wave = [item for item in data if remaining[item] == 0]
    done = 0
    while wave:
        wave.sort(key=position.__getitem__)
        ordered = set(wave)
        yield ordered
        done += len(wave)
        nxt = []
        for item in wave:
            for child in dependents.get(item, ()):
                remaining[child] -= 1
                if remaining[child] == 0:
                    nxt.append(child)
        wave = nxt
    if done != len(data):
        emitted = {item for item, n in remaining.items() if n == 0}
        raise CircularDependencyError({item: (deps - emitted) for item, deps in data.items()
                                       if item not in emitted})
