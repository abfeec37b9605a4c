"""Point-wise activations on sparse features
(reference: source/spira/nn/activations.py:8-18)."""
import torch

from ..tensors import SparseTensor
from ..utils.apply import fapply
from .fusion import absorbed

__all__ = ["ReLU", "ReLU6", "LeakyReLU"]


class ReLU(torch.nn.ReLU):
    def forward(self, input: SparseTensor) -> SparseTensor:
        if absorbed(self):  # applied by the preceding conv's fused epilogue
            return input
        return fapply(input, super().forward)


class ReLU6(torch.nn.ReLU6):
    def forward(self, input: SparseTensor) -> SparseTensor:
        return fapply(input, super().forward)


class LeakyReLU(torch.nn.LeakyReLU):
    def forward(self, input: SparseTensor) -> SparseTensor:
        return fapply(input, super().forward)
