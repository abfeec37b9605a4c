"""spira_amd -- MI355X-native sparse convolution with the spira Python API.

Public surface (same names and behaviour as the reference package
``spira``, source/spira/__init__.py:1-6): ``SparseTensor``, ``cat``,
``nn`` (``SparseConv``, ``KernelMapCache``, pointwise modules),
``set_kernel_map_cache`` and ``tune``.
"""
from .utils.helpers import set_kernel_map_cache, tune
from .tensors import SparseTensor
from . import nn
from . import utils
from .operators import cat

__all__ = ["SparseTensor", "cat", "nn", "utils", "set_kernel_map_cache", "tune"]
