"""Module base (autodiff/nn/module.py).

A module collects the Tensors assigned to its attributes (alone, or a list
or tuple whose first item is a Tensor) as parameters, and the modules
assigned to its attributes (alone, or in a list or tuple) as submodules.
``parameters()`` merges the submodules' parameters in and returns the
collection as a list.

The collection is a ``set`` of Tensors hashed by id, as in the reference:
its iteration order -- a function of the ids and of the order they were
added -- is the order in which an optimizer traces its updates, which fixes
the ids of every update node.  Parameters are added in the same sequence as
the reference adds them."""
from ..graph.tensor import Tensor

__all__ = ["Module"]


class Module:
    def __init__(self):
        object.__setattr__(self, "_parameters", set())
        object.__setattr__(self, "_modules", [])

    def __setattr__(self, name, value):
        group = value if isinstance(value, (list, tuple)) else (value,)
        if group and isinstance(group[0], Tensor):
            self._adopt(group)
        elif group and isinstance(group[0], Module):
            self._modules.extend(group)
        object.__setattr__(self, name, value)

    def _adopt(self, tensors):
        """Add the tensors whose id is not already collected (checked
        against the collection as it was before this call)."""
        known = {p.id for p in self._parameters}
        for t in tensors:
            if t.id not in known:
                self._parameters.add(t)

    def parameters(self):
        for sub in self._modules:
            self._adopt(sub.parameters())
        return list(self._parameters)

    def __call__(self, *args, **kwargs):
        return self.forward(*args, **kwargs)

    def forward(self, *args, **kwargs):
        raise NotImplementedError(f"{type(self).__name__} defines no forward()")
