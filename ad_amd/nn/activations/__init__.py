"""Activation modules (autodiff/nn/activations/)."""
from ..module import Module

__all__ = ["ReLU", "Sigmoid"]


class ReLU(Module):
    def forward(self, x):
        return x.relu()


class Sigmoid(Module):
    def forward(self, x):
        return x.sigmoid()
