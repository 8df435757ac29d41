"""Chain of modules (autodiff/nn/sequential.py:6-16)."""
from ..node import Node  # noqa: F401
from .module import Module

__all__ = ["Sequential", "Node"]


class Sequential(Module):
    def __init__(self, *args, **kwargs):
        super().__init__()
        for a in args:
            assert isinstance(a, Module), "not a seq module!"
        self.modules = args

    def __call__(self, x):
        for mod in self.modules:
            x = mod(x)
        return x
