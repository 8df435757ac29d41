"""Plain SGD as in-place graph updates (autodiff/nn/optimizers/SGD.py:4-21).
``step`` replaces each list entry with its in-place update node."""
from ...graph.tensor import Tensor

__all__ = ["SGD"]


class SGD:
    def __init__(self, parameters, lr=0.001):
        self.parameters = parameters
        self.lr = lr
        for p in self.parameters:
            p.requires_grad = True

    def step(self):
        for idx in range(len(self.parameters)):
            if isinstance(self.parameters[idx], Tensor):
                self.parameters[idx] -= self.lr * self.parameters[idx].grad()

    def zero_grad(self):
        for idx in range(len(self.parameters)):
            if isinstance(self.parameters[idx], Tensor):
                self.parameters[idx].grad_tensor = None
