"""Sparse tensor container (reference: source/spira/tensors.py:10-65)."""
from __future__ import annotations

from typing import List, Optional, Tuple, Union

import torch

from .utils.helpers import as_tuple

__all__ = ["SparseTensor"]


class SparseTensor:
    """Voxel coordinates plus per-voxel features.

    ``coordinates`` start as raw ``[N, 3] int32`` voxels; ``order()`` replaces
    them with sorted packed keys (``int64`` when ``double`` else ``int32``) and
    permutes the features to match.  ``stride`` is the per-axis tensor stride.
    """

    def __init__(self, coordinates: torch.Tensor, features: Optional[torch.Tensor],
                 stride: Union[int, Tuple[int, ...]] = 1, double: bool = False):
        self._coordinates = coordinates
        self._feats = features
        # a channel concatenation not yet materialised (spira_amd.cat): the
        # output-stationary kernels gather straight from the two parts
        self._parts: Optional[List[torch.Tensor]] = None
        self._double = double
        self._stride = as_tuple(stride, size=3, name="strides")

    @property
    def _features(self) -> torch.Tensor:
        if self._feats is None and self._parts is not None:
            self._feats = torch.cat(self._parts, dim=1)
            self._parts = None
        return self._feats

    @_features.setter
    def _features(self, value: torch.Tensor) -> None:
        self._feats = value
        self._parts = None

    @classmethod
    def _concatenated(cls, parts: List[torch.Tensor], coordinates: torch.Tensor,
                      stride: Union[int, Tuple[int, ...]]) -> "SparseTensor":
        t = cls(coordinates=coordinates, features=None, stride=stride)
        t._parts = list(parts)
        return t

    @property
    def coordinates(self) -> torch.Tensor:
        return self._coordinates

    @property
    def features(self) -> torch.Tensor:
        return self._features

    @property
    def stride(self) -> Tuple[int, int, int]:
        return self._stride

    def cuda(self) -> "SparseTensor":
        self._coordinates = self._coordinates.cuda()
        self._features = self._features.cuda()
        return self

    def to(self, dtype) -> "SparseTensor":
        self._features = self._features.to(dtype=dtype)
        return self

    def half(self) -> "SparseTensor":
        self._features = self._features.half()
        return self

    def contiguous(self) -> "SparseTensor":
        self._coordinates = self._coordinates.contiguous()
        self._features = self._features.contiguous()
        return self

    def __add__(self, other: "SparseTensor") -> "SparseTensor":
        return SparseTensor(coordinates=self._coordinates, features=self._features + other._features,
                            stride=self._stride)

    def order(self) -> "SparseTensor":
        """Pack and sort the coordinates; features follow the sort."""
        from .nn.functional._native import _C
        from .nn.functional.indexing import _require_gpu

        coordinates = self._coordinates.contiguous()
        _require_gpu(coordinates)
        # (the int32 permutation indexes directly: no int64 copy of it)
        keys, index = _C.cuda_flatten_sort(coordinates, self._double)
        self._coordinates = keys
        self._features = self._features.index_select(0, index)
        return self
