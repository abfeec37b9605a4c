"""Apply a feature-wise function to a sparse tensor
(reference: source/spira/utils/apply.py:10-18)."""
from typing import Callable

import torch

from ..tensors import SparseTensor

__all__ = ["fapply"]


def fapply(input: SparseTensor, fn: Callable[..., torch.Tensor], *args, **kwargs) -> SparseTensor:
    return SparseTensor(features=fn(input._features, *args, **kwargs), coordinates=input._coordinates,
                        stride=input._stride)
