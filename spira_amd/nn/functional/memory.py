"""Buffer utilities (reference: source/spira/nn/functional/memory.py:7-11)."""
from ._native import _C

__all__ = ["cuda_free_buffers", "cuda_reset_error"]


def cuda_free_buffers():
    return _C.cuda_free_buffers()


def cuda_reset_error():
    _C.cuda_reset_error()
