"""Tensor-level operators (reference: source/spira/operators.py:11-13)."""
from __future__ import annotations

from typing import List

import torch

from .tensors import SparseTensor

__all__ = ["cat"]


def cat(inputs: List[SparseTensor]) -> SparseTensor:
    """Channel concatenation for skip connections; coordinates and stride of
    the first input are kept.  Two fp16 GPU parts whose split falls on a
    32-channel block (and that need no gradient) are not copied: the
    result's features materialise on first access, and the output-stationary
    convolutions gather from the parts directly."""
    feats = [x._features for x in inputs]
    if (len(feats) == 2 and all(f.is_cuda and f.dtype == torch.float16 and f.dim() == 2 for f in feats)
            and feats[0].shape[0] == feats[1].shape[0] and feats[0].shape[1] % 32 == 0
            and feats[1].shape[1] % 8 == 0
            and not (torch.is_grad_enabled() and any(f.requires_grad for f in feats))):
        return SparseTensor._concatenated([f.contiguous() for f in feats], inputs[0]._coordinates,
                                          inputs[0]._stride)
    return SparseTensor(features=torch.cat(feats, dim=1), coordinates=inputs[0]._coordinates,
                        stride=inputs[0]._stride)
