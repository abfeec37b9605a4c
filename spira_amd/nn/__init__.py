from .conv import SparseConv, KernelMapCache
from .activations import ReLU, ReLU6, LeakyReLU
from .normalizations import BatchNorm

__all__ = ["SparseConv", "KernelMapCache", "ReLU", "ReLU6", "LeakyReLU", "BatchNorm"]
