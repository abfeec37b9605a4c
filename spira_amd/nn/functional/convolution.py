"""Feature dataflows (reference: source/spira/nn/functional/convolution.py:1-177).

``gather_tile_size`` / ``scatter_tile_size`` / ``parallel`` are accepted for
API compatibility; the gfx950 kernels pick their own tiling and run the
per-offset GEMMs as one grouped launch.
"""
from __future__ import annotations

from typing import Optional

import torch

from ._native import _C

__all__ = [
    "cuda_time_gather", "cuda_time_scatter", "sparse_convolution_forward_ws",
    "sparse_convolution_forward_ws_merged", "sparse_convolution_forward_os",
    "sparse_convolution_forward_hs", "sparse_convolution_forward_hs_merged", "cuda_time_gemm",
    "set_gemm_parallel_level", "dense_forward",
]

GEMM_PARALLEL_LEVEL = 4


def set_gemm_parallel_level(level: int):
    global GEMM_PARALLEL_LEVEL
    GEMM_PARALLEL_LEVEL = level


def _c(t: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    return None if t is None else t.contiguous()


def cuda_time_gather(weights, source_masks, target_masks, kernel_map_sizes, tile_size: int,
                     is_hybrid: bool = False, threshold: Optional[float] = 0) -> float:
    return _C.cuda_time_gather(tile_size, threshold, is_hybrid, _c(weights), _c(source_masks), _c(target_masks),
                               _c(kernel_map_sizes))


def cuda_time_scatter(weights, source_masks, target_masks, kernel_map_sizes, tile_size: int,
                      is_hybrid: bool = False, threshold: Optional[float] = 0) -> float:
    return _C.cuda_time_scatter(tile_size, threshold, is_hybrid, _c(weights), _c(source_masks), _c(target_masks),
                                _c(kernel_map_sizes))


def cuda_time_gemm(weights, source_masks, target_masks, kernel_map_sizes, parallel: Optional[int] = None,
                   is_hybrid: bool = False, threshold: Optional[float] = 0) -> float:
    if parallel is None:
        parallel = GEMM_PARALLEL_LEVEL
    return _C.cuda_time_gemm(parallel, threshold, is_hybrid, _c(weights), _c(source_masks), _c(target_masks),
                             _c(kernel_map_sizes))


def _gpu(sources: torch.Tensor) -> None:
    if not sources.is_cuda:
        raise NotImplementedError("spira_amd runs on the GPU only")


def _epi(epilogue) -> tuple:
    """(scale, shift, residual, relu) folded into the output write:
    y = conv * scale[c] + shift[c] + residual[t, c], then max(y, 0) if relu.
    scale / shift are fp32 [C_out], residual is [T, C_out] in the feature
    dtype; None entries are skipped.  No reference counterpart: the
    reference applies batch norm, ReLU and the residual add as separate ops
    (scripts/models/spira/modules/blocks.py:12-84)."""
    if epilogue is None:
        return (None, None, None, False)
    scale, shift, residual, relu = epilogue
    return (_c(scale), _c(shift), _c(residual), bool(relu))


def sparse_convolution_forward_ws(num_sources: int, num_targets: int, sources, weights, source_masks,
                                  target_masks, kernel_map_sizes, gather_tile_size: int, scatter_tile_size: int,
                                  parallel: Optional[int] = None, threshold: Optional[float] = 0, *, epilogue=None):
    _gpu(sources)
    if parallel is None:
        parallel = GEMM_PARALLEL_LEVEL
    return _C.cuda_sparse_convolution_forward_ws(num_sources, num_targets, gather_tile_size, scatter_tile_size,
                                                 parallel, threshold, _c(sources), _c(weights), _c(source_masks),
                                                 _c(target_masks), _c(kernel_map_sizes), *_epi(epilogue))


def sparse_convolution_forward_ws_merged(num_sources: int, num_targets: int, sources, weights, naddrs, qnaddrs,
                                         nbmaps, mapsize: int, qmapsize: int, transpose: Optional[bool] = False, *,
                                         epilogue=None):
    _gpu(sources)
    return _C.cuda_sparse_convolution_forward_ws_merged(num_sources, num_targets, _c(sources), _c(weights),
                                                        _c(naddrs), _c(qnaddrs), _c(nbmaps), mapsize, qmapsize,
                                                        bool(transpose), *_epi(epilogue))


def sparse_convolution_forward_hs(num_sources: int, num_targets: int, sources, weights, source_masks,
                                  target_masks, kernel_map_sizes, out_in_map, gather_tile_size: int,
                                  scatter_tile_size: int, parallel: Optional[int] = None,
                                  threshold: Optional[float] = 0, *, epilogue=None):
    _gpu(sources)
    if parallel is None:
        parallel = GEMM_PARALLEL_LEVEL
    return _C.cuda_sparse_convolution_forward_hs(num_sources, num_targets, gather_tile_size, scatter_tile_size,
                                                 parallel, threshold, _c(sources), _c(weights), _c(source_masks),
                                                 _c(target_masks), _c(kernel_map_sizes), _c(out_in_map),
                                                 *_epi(epilogue))


def sparse_convolution_forward_hs_merged(num_sources: int, num_targets: int, sources, weights, naddrs, qnaddrs,
                                         nbmaps, out_in_map, mapsize: int, qmapsize: int,
                                         transpose: Optional[bool] = False, *, epilogue=None):
    _gpu(sources)
    return _C.cuda_sparse_convolution_forward_hs_merged(num_sources, num_targets, _c(sources), _c(weights),
                                                        _c(naddrs), _c(qnaddrs), _c(nbmaps), _c(out_in_map),
                                                        mapsize, qmapsize, bool(transpose), *_epi(epilogue))


def _tuning(tuning) -> Optional[tuple]:
    """An output-stationary launch choice: None (automatic) or a tuple
    (col_tile, step_channels, offset_splits, offset_pack, block_order,
    row_order[, row_walk[, balance_offsets[, blocks_per_cu]]]); 0 (and -1
    for row_order) in a field = automatic; row_walk 1 sums each target's
    valid pairs on the vector ALU (fp16 layers of at most 16 input
    channels); balance_offsets > 0 splits a row tile of a row-ordered map
    with more valid offsets than that over several blocks (-1: never);
    blocks_per_cu 1..8 caps the resident blocks per CU (-1: no cap)."""
    if tuning is None:
        return None
    if type(tuning) is tuple:
        t = _TUNINGS.get(tuning)
        if t is not None:
            return t
    t = tuple(int(v) for v in tuning)
    if len(t) not in (6, 7, 8, 9):
        raise ValueError(f"an output-stationary tuning has 6 to 9 fields, got {len(t)}")
    if type(tuning) is tuple and len(_TUNINGS) < 4096:
        _TUNINGS[tuning] = t
    return t


# tunings already checked (a layer passes the same tuple on every call)
_TUNINGS: dict = {}


def dense_forward(sources, weights, *, epilogue=None, sources2=None, tuning=None):
    """sources @ weights[0] (a 1x1x1, stride-1 layer) with the fused epilogue,
    on the output-stationary kernel with the identity map (reference: the
    torch.mm path of SparseConv.forward, source/spira/nn/conv.py:310-313).
    ``sources2``: the input is the channel concatenation [sources | sources2],
    gathered from its two parts without materialising it."""
    _gpu(sources)
    return _C.cuda_dense_forward(_c(sources), _c(weights), *_epi(epilogue), _c(sources2), _tuning(tuning))


def sparse_convolution_forward_os(num_sources: int, num_targets: int, out_in_map, sources, weights, *,
                                  epilogue=None, sources2=None, tuning=None):
    """``sources2``: the layer input is the channel concatenation
    [sources | sources2] (a decoder's skip connection), gathered from its two
    parts without materialising it.  ``tuning``: the layer's launch choices
    (see ``_tuning``); they change the schedule, never the result."""
    _gpu(sources)
    return _C.cuda_sparse_convolution_forward_os(num_sources, num_targets, _c(out_in_map), _c(sources),
                                                 _c(weights), *_epi(epilogue), _c(sources2), _tuning(tuning))
