"""``x @ w (+ b)`` with N(0,1) init (autodiff/nn/linear.py:5-15)."""
from ..graph.tensor import Tensor
from .module import Module

__all__ = ["Linear"]


class Linear(Module):
    def __init__(self, input_dim: int, output_dim: int, bias: bool = True):
        super().__init__()
        self.w = Tensor.randn([input_dim, output_dim])
        self.b = Tensor.randn([output_dim]) if bias else None

    def forward(self, x):
        res = x @ self.w
        if self.b is not None:
            res = res + self.b
        return res
