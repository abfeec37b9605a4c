"""Coordinate and kernel-map functions
(reference: source/spira/nn/functional/indexing.py:1-105).

Kernel maps come back as the reference's 9-tuple
``(S, T, map, t3, t4, t5, t6, mapsize, qmapsize)``; see ``build_kmap``.
"""
from __future__ import annotations

from typing import List, Tuple

import torch

from ...utils.helpers import as_tuple
from ...utils.typing import ScalarOrTuple
from ._native import _C

__all__ = [
    "flat_sort", "unflatten", "downsample", "build_kmap", "convert_transposed_os", "convert_transposed_os_ordered",
    "build_kmap_streamed", "streamed_output_generate", "downsample_chain_launch", "build_kmap_no_small_z", "sparse_quantize",
    "prepare_row_order",
    "prepare_row_orders",
]


def _require_gpu(t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise NotImplementedError("spira_amd runs on the GPU only")


def sparse_quantize(points: torch.Tensor, voxel_size: ScalarOrTuple[float] = 1.0) -> torch.Tensor:
    """Voxelize ``[N, 3]`` float32 / float64 points on the GPU: floor(points /
    voxel_size), one voxel per value of the reference's coordinate hash (its
    first point), sorted lexicographically; returns ``[M, 3] int32`` (reference:
    sparse_quantize, datasets/helpers.py:14-30, which does this on the host)."""
    _require_gpu(points)
    vx, vy, vz = (float(v) for v in as_tuple(voxel_size, size=3, name="voxel_size"))
    return _C.voxelize(points, vx, vy, vz)


def flat_sort(coordinates: torch.Tensor, double: bool = False):
    """Pack ``[N, 3] int32`` voxels into keys and sort them; returns
    ``(sorted keys, permutation as int64)``."""
    coordinates = coordinates.contiguous()
    _require_gpu(coordinates)
    keys, index = _C.cuda_flatten_sort(coordinates, double)
    return keys, index.to(torch.int64)


def unflatten(coordinates: torch.Tensor) -> torch.Tensor:
    coordinates = coordinates.contiguous()
    _require_gpu(coordinates)
    return _C.cuda_unflatten(coordinates)


def streamed_output_generate(coordinates: torch.Tensor, target_strides: List[Tuple[int, int, int]]):
    coordinates = coordinates.contiguous()
    _require_gpu(coordinates)
    return _C.cuda_streamed_output_generate(coordinates, [as_tuple(s, size=3) for s in target_strides])


def downsample_chain_launch(coordinates: torch.Tensor, target_strides: List[Tuple[int, int, int]]):
    """Queue the chained downsample of sorted keys on the current stream
    without reading anything back: ``(outputs, counts)``, the outputs at full
    capacity and ``counts`` a device int32 tensor of the level counts followed
    by the unsorted-input flag; ``None`` when the strides do not chain (or no
    keys), for which :func:`streamed_output_generate` is the call."""
    coordinates = coordinates.contiguous()
    _require_gpu(coordinates)
    r = _C.cuda_downsample_chain_launch(coordinates, [as_tuple(s, size=3) for s in target_strides])
    if not r:
        return None
    return list(r[:-1]), r[-1]


def build_kmap_streamed(voxels: List[torch.Tensor], kernel_sizes: List[ScalarOrTuple[int]],
                        source_strides: List[ScalarOrTuple[int]], dataflow: List[int], begin: int = 0):
    voxels = [v.contiguous() for v in voxels]
    kernel_sizes = [as_tuple(k, size=3, name="kernel_size") for k in kernel_sizes]
    source_strides = [as_tuple(s, size=3, name="kernel_stride") for s in source_strides]
    if not (len(kernel_sizes) == len(source_strides) == len(dataflow)):
        raise ValueError("All argument lists must have the same length in build_kmap_streamed")
    return _C.cuda_binary_search_streamed(voxels, kernel_sizes, source_strides, list(dataflow), int(begin))


def prepare_row_order(kmap: torch.Tensor, num_targets: int, request: int = -1) -> List[torch.Tensor]:
    """Queue the row order of an output-stationary map on the current stream
    if the fp16 convolution kernel will walk it in row order (by default:
    large maps of 27 to 57 offsets; ``request`` 1 / 0 asks for it / against
    it), so that it is computed with the maps instead of at the first layer
    that uses it.  Returns the row order's tensors (empty if the map gets
    none)."""
    _require_gpu(kmap)
    return list(_C.prepare_row_order(kmap, int(num_targets), int(request)))


def prepare_row_orders(kmaps: List[torch.Tensor], num_targets: List[int], requests: List[int]) -> None:
    """:func:`prepare_row_order` for several maps at once: the maps of at
    most 27 offsets that take a row order are ordered by one batched chain of
    launches (one sort over all their rows) instead of one chain each."""
    for m in kmaps:
        _require_gpu(m)
    _C.prepare_row_orders(list(kmaps), [int(t) for t in num_targets], [int(r) for r in requests])


def downsample(coordinates: torch.Tensor, target_stride: Tuple[int, int, int]) -> torch.Tensor:
    coordinates = coordinates.contiguous()
    _require_gpu(coordinates)
    return _C.cuda_downsample(coordinates, *as_tuple(target_stride, size=3))


def build_kmap(sources: torch.Tensor, targets: torch.Tensor, kernel_size: ScalarOrTuple[int],
               source_stride: ScalarOrTuple[int], dataflow: int = 0):
    """Kernel map of sorted unique ``sources`` for ``targets``.

    dataflow 0: ``map [Tp, K]`` (output-stationary, z-major columns);
    1 / odd: ``map [K, Tp]``, ``nbmaps [2, P]``, ``nbsizes``, ``naddrs``,
    ``qnaddrs``, ``mapsize``, ``qmapsize``; 2 / even: ``map``,
    ``source_masks``, ``target_masks``, ``nbsizes``.  Hybrid dataflows (3-8)
    order rows dense-first by L1 distance; above 4 the first entry is the
    dense part ``[Tp, dense]``.
    """
    sources = sources.contiguous()
    targets = targets.contiguous()
    return _C.cuda_binary_search(sources, targets, as_tuple(kernel_size, size=3, name="kernel_size"),
                                 as_tuple(source_stride, size=3, name="kernel_stride"), dataflow)


def convert_transposed_os_ordered(out_in_map: torch.Tensor, num_coarse: int, input_size: int) -> torch.Tensor:
    """:func:`convert_transposed_os` with ``partition=True`` (``out_in_map``
    has ``num_coarse`` rows of targets), and the inverse's row order made in
    the same pass and kept for the fp16 convolution that walks it."""
    _require_gpu(out_in_map)
    return _C.convert_transposed_os_ordered(out_in_map.contiguous(), int(num_coarse), int(input_size))


def convert_transposed_os(out_in_map: torch.Tensor, input_size: int, partition: bool = False) -> torch.Tensor:
    """``partition``: every source is in exactly one map entry (a
    down-sampling map whose kernel equals its stride), so one pass writes
    whole rows; any other map needs the default."""
    return _C.cuda_convert_transposed_os(out_in_map.contiguous(), input_size, partition)


def build_kmap_no_small_z(sources: torch.Tensor, targets: torch.Tensor, kernel_size: ScalarOrTuple[int],
                          source_stride: ScalarOrTuple[int]):
    """Ablation: one full search per kernel offset, no z-scan; canonical columns."""
    return _C.cuda_binary_search_no_small_z(sources.contiguous(), targets.contiguous(),
                                            as_tuple(kernel_size, size=3, name="kernel_size"),
                                            as_tuple(source_stride, size=3, name="kernel_stride"))
