"""Writes the seeded inputs of the reference's known-answer tests as
fixtures, so GPU runs need no torch import.

tests/dotprod_test.py:12-15 of the reference draws its inputs with
``torch.manual_seed(42); randn(2,5); randn(5,3); randn(3)``.  Run:
``python tests/golden/make_inputs.py`` (needs torch, CPU only)."""
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def main():
    import torch
    torch.manual_seed(42)
    inp = torch.randn(2, 5).numpy()
    weight = torch.randn(5, 3).numpy()
    bias = torch.randn(3).numpy()
    np.savez(os.path.join(HERE, "dotprod_test_inputs.npz"), inp=inp, weight=weight, bias=bias)


if __name__ == "__main__":
    main()
