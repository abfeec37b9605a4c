"""Batch normalisation on sparse features
(reference: source/spira/nn/normalizations.py:8-10)."""
import torch

from ..tensors import SparseTensor
from ..utils.apply import fapply

__all__ = ["BatchNorm"]


class BatchNorm(torch.nn.BatchNorm1d):
    def forward(self, input: SparseTensor) -> SparseTensor:
        return fapply(input, super().forward)
