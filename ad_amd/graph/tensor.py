"""Leaf value with host data (autodiff/graph/tensor.py).  Its buffer is
initialised from ``arr`` (float32) and, after execution, ``arr`` holds the
device's final values.  ``grad()`` is the node of its accumulated gradient
once a loss has been differentiated."""
import numpy as np

from ..node import Node

__all__ = ["Tensor"]


class Tensor(Node):
    def __init__(self, arr, requires_grad: bool = False):
        super().__init__([], list(arr.shape))
        self.arr = arr.astype(np.float32)
        self.grad_tensor = None
        self.requires_grad = requires_grad

    def grad(self):
        if self.grad_tensor is None:
            raise RuntimeError(f"tensor {self.id} has no gradient: call .backward() on a loss that uses it")
        return self.grad_tensor

    def __repr__(self) -> str:
        return f"Tensor(id: {self.id}, orig_shape: {self.shape})"

    def repeat_helper(self, is_child):
        return ("Tensor", self.id)

    @classmethod
    def from_torch(cls, arr, requires_grad: bool = False):
        return cls(arr.numpy(), requires_grad=requires_grad)

    @classmethod
    def randn(cls, shape, requires_grad=False):
        return cls(np.random.randn(*shape), requires_grad)

    @classmethod
    def fill(cls, val: float, shape, requires_grad=False):
        return cls(np.full(tuple(shape), val), requires_grad)

    @classmethod
    def ones(cls, shape, requires_grad=False):
        return cls.fill(1.0, shape, requires_grad)

    @classmethod
    def zeros(cls, shape, requires_grad=False):
        return cls.fill(0.0, shape, requires_grad)
