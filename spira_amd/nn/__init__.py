from .conv import SparseConv, KernelMapCache
from .activations import ReLU, ReLU6, LeakyReLU
from .normalizations import BatchNorm
from .fusion import fuse_epilogues

__all__ = ["SparseConv", "KernelMapCache", "ReLU", "ReLU6", "LeakyReLU", "BatchNorm", "fuse_epilogues"]
