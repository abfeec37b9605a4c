"""Tensor-level operators (reference: source/spira/operators.py:11-13)."""
from __future__ import annotations

from typing import List

import torch

from .tensors import SparseTensor

__all__ = ["cat"]


def cat(inputs: List[SparseTensor]) -> SparseTensor:
    """Channel concatenation for skip connections; coordinates and stride of
    the first input are kept."""
    feats = torch.cat([x._features for x in inputs], dim=1)
    return SparseTensor(features=feats, coordinates=inputs[0]._coordinates, stride=inputs[0]._stride)
