"""Module base (autodiff/nn/module.py:5-43).  Parameters are kept in a set of
Tensors (hashed by id), and ``parameters()`` returns that set as a list, so
the optimizer's update order is the set's iteration order."""
from typing import List, Tuple

from ..graph.tensor import Tensor

__all__ = ["Module"]


class Module:
    def __init__(self):
        self._parameters = set()
        self._modules = []

    def _add_to_params(self, nodes):
        current_ids = set({p.id for p in self._parameters})
        for n in nodes:
            if not (n.id in current_ids):
                self._parameters.add(n)

    def __setattr__(self, name, value):
        if isinstance(value, Tensor):
            self._add_to_params([value])
        elif isinstance(value, List) and len(value) > 0 and isinstance(value[0], Tensor):
            self._add_to_params(value)
        elif isinstance(value, Tuple) and len(value) > 0 and isinstance(value[0], Tensor):
            self._add_to_params(value)
        elif isinstance(value, Module):
            self._modules.append(value)
        elif isinstance(value, List) and len(value) > 0 and isinstance(value[0], Module):
            self._modules.extend(value)
        elif isinstance(value, Tuple) and len(value) > 0 and isinstance(value[0], Module):
            self._modules.extend(value)
        super().__setattr__(name, value)

    def parameters(self):
        for m in self._modules:
            self._add_to_params(m.parameters())
        return list(self._parameters)

    def __call__(self, *args, **kwargs):
        return self.forward(*args, **kwargs)

    def forward(self, *args, **kwargs):
        raise NotImplementedError("You must override forward()")
