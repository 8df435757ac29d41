"""Leaf tensor holding host data (autodiff/graph/tensor.py:11-64)."""
import numpy as np

from ..node import Node

__all__ = ["Tensor"]


class Tensor(Node):
    def __init__(self, arr, requires_grad: bool = False):
        super().__init__([], list(arr.shape))
        self.arr = arr.astype(np.float32)
        self.grad_tensor = None
        self.requires_grad = requires_grad

    def _bck(self, grad):
        if not isinstance(grad, Node):
            raise TypeError("Backward on tensor grad is not tensoor")
        if self.requires_grad:
            if self.grad_tensor is None:
                self.grad_tensor = grad
            else:
                self.grad_tensor += grad     # an in-place ADD node
        return None

    def grad(self):
        if self.grad_tensor is None:
            raise RuntimeError(f"Gradient on tensor {self.id} is none! Make sure you call .backward()")
        return self.grad_tensor

    def repeat_helper(self, is_child):
        return ("Tensor", self.id)

    def __repr__(self) -> str:
        return f"Tensor(id: {self.id}, orig_shape: {self.shape})"

    @staticmethod
    def from_torch(arr, requires_grad: bool = False):
        return Tensor(arr.numpy(), requires_grad=requires_grad)

    @staticmethod
    def randn(shape, requires_grad=False):
        return Tensor(np.random.randn(*shape), requires_grad)

    @staticmethod
    def fill(val: float, shape, requires_grad=False):
        return Tensor(np.full(tuple(shape), val), requires_grad)

    @staticmethod
    def ones(shape, requires_grad=False):
        return Tensor.fill(1.0, shape, requires_grad)

    @staticmethod
    def zeros(shape, requires_grad=False):
        return Tensor.fill(0.0, shape, requires_grad)
