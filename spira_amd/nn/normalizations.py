"""Batch normalisation on sparse features
(reference: source/spira/nn/normalizations.py:8-10)."""
import torch

from ..tensors import SparseTensor
from ..utils.apply import fapply
from .fusion import absorbed

__all__ = ["BatchNorm"]


class BatchNorm(torch.nn.BatchNorm1d):
    def forward(self, input: SparseTensor) -> SparseTensor:
        if absorbed(self):  # applied by the preceding conv's fused epilogue
            return input
        return fapply(input, super().forward)
