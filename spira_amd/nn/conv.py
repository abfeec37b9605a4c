"""Sparse convolution layer and the kernel-map cache
(reference: source/spira/nn/conv.py:17-419).

Dataflow numbering (``_tunable_config['map_dataflow']``):
  0      output-stationary implicit GEMM (map [Tp, K], z-major weight rows)
  1      fused weight-stationary over compacted pairs (canonical weight rows)
  2      gather -> GEMM -> scatter over masks (canonical weight rows)
  3..8   hybrid: offsets with L1 < (d-1)//2 output-stationary, the rest
         weight-stationary (odd: fused, even: gather-scatter); weight rows
         ordered dense-first
``force_os`` runs a weight-stationary map output-stationary by transposing
it (canonical weight rows).  Transposed layers reuse the map of the matching
downsampling layer with sources and targets swapped.
"""
from __future__ import annotations

import contextlib
import operator
from typing import Any, Dict, List, Optional, Tuple, Union

import numpy as np
import torch
from torch.nn import Module

from ..tensors import SparseTensor
from ..utils.helpers import as_tuple
from ..utils.typing import ScalarOrTuple
from . import functional as F
from .fusion import bn_affine

__all__ = ["SparseConv", "KernelMapCache"]


class KernelMapCache:
    """Coordinates per tensor stride and kernel maps per
    ``(source stride, target stride, kernel size)``."""

    #: queue the row orders of the large output-stationary maps with the
    #: network-wide map build (only the fp16 convolution kernel uses them; a
    #: network run in fp32 can turn this off to skip that work)
    prepare_row_orders = True

    def __init__(self):
        self._kernel_maps_cache: Dict[tuple, list] = {}
        self._coordinates_cache: Dict[tuple, torch.Tensor] = {}
        #: per map key (source stride, target stride, kernel size): walk the
        #: output-stationary map in row order (1) or not (0); maps without an
        #: entry follow the library's default rule.  Set by the selector.
        self.row_order_requests: Dict[tuple, int] = {}

    def reset(self) -> None:
        self._coordinates_cache.clear()
        self._kernel_maps_cache.clear()

    def get_target_coordinates(self, source_coordinates: torch.Tensor, source_stride: ScalarOrTuple[int],
                               target_stride: ScalarOrTuple[int], transposed: bool = False) -> torch.Tensor:
        source_stride = as_tuple(source_stride, size=3, name="source_stride")
        target_stride = as_tuple(target_stride, size=3, name="target_stride")
        self._coordinates_cache.setdefault(source_stride, source_coordinates)
        if target_stride in self._coordinates_cache:
            return self._coordinates_cache[target_stride]
        if transposed:
            raise RuntimeError("Layer must transpose=True must have its corresponding "
                               "non-transposed layer before its execution")
        target = F.downsample(source_coordinates, target_stride)
        self._coordinates_cache[target_stride] = target
        return target

    def get_kernel_map(self, source_coordinates: torch.Tensor, source_stride: ScalarOrTuple[int],
                       target_coordinates: torch.Tensor, target_stride: ScalarOrTuple[int],
                       kernel_size: ScalarOrTuple[int], map_dataflow: int, force_os: bool = False,
                       transposed: bool = False):
        source_stride = as_tuple(source_stride, size=3, name="source_stride")
        target_stride = as_tuple(target_stride, size=3, name="target_stride")
        kernel_size = as_tuple(kernel_size, size=3, name="kernel_size")
        key = ((target_stride, source_stride) if transposed else (source_stride, target_stride)) + (kernel_size,)

        entry = self._kernel_maps_cache.get(key)
        if entry is not None:
            # entry = [transposed-to-[Tp, K] flag, S, T, map, ...]
            if force_os and not entry[0]:
                entry[3] = entry[3].T.contiguous()
                entry[0] = True
            if (map_dataflow == 0 or force_os) and transposed:
                out = list(entry[1:])
                # The forward map's sources are at target_stride (fine), its
                # targets at source_stride (coarse, the down-sampled
                # sources).  With a kernel of 2 (offsets 0 and 1) or 1 per
                # axis equal to the stride ratio, each fine voxel lies in
                # exactly one entry, that of its own coarse cell.
                part = all(k in (1, 2) and c == k * f for f, c, k in zip(target_stride, source_stride, kernel_size))
                if part:
                    # (with its row order, made in the same pass)
                    out[2] = F.convert_transposed_os_ordered(entry[3], entry[2], entry[1])
                else:
                    out[2] = F.convert_transposed_os(entry[3], entry[1])
                return out
            return entry[1:]

        if transposed:
            raise RuntimeError("Layer must transpose=True must have its corresponding "
                               "non-transposed layer before its execution")
        kmap = F.build_kmap(source_coordinates, target_coordinates, kernel_size, source_stride, map_dataflow)
        entry = [False, *kmap]
        if force_os:
            entry[3] = entry[3].T.contiguous()
            entry[0] = True
        self._kernel_maps_cache[key] = entry
        return entry[1:]

    def add_all_kernel_maps(self, source_coordinates: torch.Tensor, kernel_sizes: List[ScalarOrTuple[int]],
                            source_strides: List[ScalarOrTuple[int]], target_strides: List[ScalarOrTuple[int]],
                            init_stride: Union[int, Tuple[int, ...]], dataflow: List[int]) -> "KernelMapCache":
        """Network-wide precompute: all downsampled coordinate sets, then every
        layer map concurrently (map i: sources voxels[i//2], targets
        voxels[(i+1)//2])."""
        src_strides = list(source_strides)[:-1]
        s_stride = as_tuple(init_stride, size=3)
        map_keys = []
        s_prev = s_stride
        for i in range(len(kernel_sizes)):
            t_stride = as_tuple(source_strides[i + 1], size=3)
            map_keys.append((s_prev, t_stride, as_tuple(kernel_sizes[i], size=3)))
            s_prev = t_stride


        # Map 0 (voxels[0] to voxels[0]) needs no downsampled level: it is
        # queued between the chained downsample and the host read of the
        # level counts, so that the GPU works on it while the host waits.
        kmaps, outputs = [], None
        launched = F.downsample_chain_launch(source_coordinates, target_strides) if kernel_sizes else None
        if launched is not None:
            levels, counts = launched
            host = torch.empty(counts.numel(), dtype=torch.int32, pin_memory=True)
            host.copy_(counts, non_blocking=True)
            ready = torch.cuda.Event()
            ready.record()
            kmaps = F.build_kmap_streamed([source_coordinates], kernel_sizes[:1], src_strides[:1], dataflow[:1])
            ready.synchronize()
            n = host.tolist()
            if n[-1] == 0:
                outputs = [lv[:c] for lv, c in zip(levels, n[:-1])]
        if outputs is None:  # strides that do not chain, or unsorted keys
            outputs = F.streamed_output_generate(source_coordinates, target_strides)
        voxels = [source_coordinates] + list(outputs)
        self._coordinates_cache[s_stride] = voxels[0]
        for i, ts in enumerate(target_strides):
            self._coordinates_cache[as_tuple(ts, size=3)] = voxels[i + 1]
        first = len(kmaps)
        kmaps += F.build_kmap_streamed(voxels, kernel_sizes, src_strides, dataflow, begin=first)
        # the row orders of the large output-stationary maps, all in one
        # batched chain of launches
        if self.prepare_row_orders:
            sel = [i for i in range(len(kernel_sizes)) if dataflow[i] == 0]
            if sel:
                F.prepare_row_orders([kmaps[i][2] for i in sel], [kmaps[i][1] for i in sel],
                                     [self.row_order_requests.get(map_keys[i], -1) for i in sel])
        for i in range(len(kernel_sizes)):
            t_stride = as_tuple(source_strides[i + 1], size=3)
            self._kernel_maps_cache[(s_stride, t_stride, as_tuple(kernel_sizes[i], size=3))] = [False, *kmaps[i]]
            s_stride = t_stride
        return self


class SparseConv(Module):
    __AVAILABLE_THRESHOLD__ = [-1, *list(np.linspace(0, 2, num=50)), None]
    __NUM_TUNING_ROUNDS__ = 5

    def __init__(self, in_channels: int, out_channels: int, kernel_size: ScalarOrTuple[int],
                 stride: ScalarOrTuple[int] = 1, bias: bool = False, transposed: bool = False):
        super().__init__()
        self.in_channels = in_channels
        self.out_channels = out_channels
        self.kernel_size = as_tuple(kernel_size, size=3, name="kernel_size")
        self.stride = as_tuple(stride, size=3, name="stride")
        self.transposed = transposed
        volume = int(np.prod(self.kernel_size))
        self.kernel = torch.nn.Parameter(torch.empty(volume, in_channels, out_channels))
        if bias:
            self.bias = torch.nn.Parameter(torch.empty(out_channels))
        else:
            self.register_parameter("bias", None)
        self.reset_parameters()
        self._kernel_map_cache: Optional[KernelMapCache] = None
        self._tunable_config: Dict[str, Any] = {
            "threshold": -1,
            "gather_tile_size": min(in_channels, 16),
            "scatter_tile_size": min(out_channels, 16),
            "map_dataflow": 2,
            "force_os": False,
            # output-stationary launch choices (col_tile, step_channels,
            # offset_splits, offset_pack, block_order, row_order); None =
            # automatic
            "os_tuning": None,
        }
        self._tuning_data = None
        self._os_tuning_data = None
        # fused epilogue (spira_amd.nn.fusion): an absorbed eval-mode batch
        # norm (plain attribute, not a submodule) and ReLU
        object.__setattr__(self, "_epi_bn", None)
        self._epi_relu = False
        # output stride per (input stride, stride, transposed)
        self._out_strides: Dict[tuple, tuple] = {}

    def _fused_active(self) -> bool:
        """The fused epilogue applies: autograd off and, with a batch norm,
        the norm in eval mode."""
        if self._epi_bn is None and not self._epi_relu:
            return False
        return not torch.is_grad_enabled() and (self._epi_bn is None or not self._epi_bn.training)

    @property
    def tunable_config(self) -> Dict[str, Any]:
        return self._tunable_config

    def reset_parameters(self) -> None:
        fan = self.out_channels if self.transposed else self.in_channels
        bound = 1.0 / np.sqrt(fan * len(self.kernel))
        self.kernel.data.uniform_(-bound, bound)
        if self.bias is not None:
            self.bias.data.uniform_(-bound, bound)

    def set_kernel_map_cache(self, cache: KernelMapCache) -> None:
        self._kernel_map_cache = cache

    @property
    def is_trivial(self) -> bool:
        return self.stride == (1, 1, 1) and self.kernel_size == (1, 1, 1)

    @contextlib.contextmanager
    def tune_gs(self, free_buffers: bool = True):
        """Record (masks, sizes) of gather-scatter runs while inside, then sweep
        the bucket threshold by timing the grouped GEMM (reference
        conv.py:217-307).  The reference's gather / scatter tile sweep has no
        counterpart here: the gather and scatter kernels of this build have
        no tile parameter (the keys stay in the config for file
        compatibility); the CDNA4 launch choices are swept by ``tune_os``."""
        try:
            self._tuning_data = []
            if free_buffers:
                F.cuda_free_buffers()
            yield
            if free_buffers:
                F.cuda_free_buffers()
            if self.is_trivial or not self._tuning_data:
                return
            best = None
            for thr in self.__AVAILABLE_THRESHOLD__:
                try:
                    t = [F.cuda_time_gemm(threshold=thr, weights=self.kernel, source_masks=sm, target_masks=tm,
                                          kernel_map_sizes=nb)
                         for _ in range(self.__NUM_TUNING_ROUNDS__) for sm, tm, nb in self._tuning_data]
                except RuntimeError:
                    F.cuda_reset_error()
                    break
                t = float(np.average(t))
                if best is None or t < best:
                    best, self._tunable_config["threshold"] = t, thr
            if free_buffers:
                F.cuda_free_buffers()
        finally:
            self._tuning_data = None

    @contextlib.contextmanager
    def tune_os(self, reps: int = 10):
        """Record the output-stationary calls made while inside, then choose
        this layer's launch choices -- column tile, step channels, offset
        splits and offset packing -- by timing the recorded calls on the
        kernel, one field at a time over two passes (the CDNA4 counterpart of
        the reference's gather / scatter tile sweep, conv.py:217-307).  The
        row order field is left as it is: it is decided per map (its sort is
        shared by every layer on the map), by ``spira_amd.utils.helpers``."""
        try:
            self._os_tuning_data = []
            yield
            data = self._os_tuning_data
            if data and self.kernel.is_cuda and self.kernel.dtype == torch.float16:
                self._tunable_config["os_tuning"] = choose_os_tuning(self, data, reps)
        finally:
            self._os_tuning_data = None

    def forward(self, inputs: SparseTensor, residual: Optional[SparseTensor] = None) -> SparseTensor:
        """residual (fused res blocks only): features added after the batch
        norm and before the ReLU of the fused epilogue."""
        # (attributes read once: a module's parameters are looked up through
        # nn.Module.__getattr__, and this runs once per layer and step)
        cfg = self._tunable_config
        d = cfg["map_dataflow"]
        force_os = cfg["force_os"]
        trivial = self.is_trivial
        kernel, bias = self.kernel, self.bias
        # an unmaterialised channel concatenation (spira_amd.cat) goes to the
        # output-stationary kernels as its two parts
        parts = inputs._parts
        if parts is not None and (trivial or d == 0 or force_os):
            x, x2 = parts
        else:
            x, x2 = inputs._features, None
        epilogue = None
        epilogue_done = False
        if self._fused_active():
            scale, shift = bn_affine(self._epi_bn) if self._epi_bn is not None else (None, None)
            if bias is not None:
                b = bias.float()
                shift = b * scale + shift if scale is not None else b
            epilogue = (scale, shift, None if residual is None else residual._features, self._epi_relu)
        elif residual is not None:
            raise ValueError("a residual is only taken by a conv with an active fused epilogue")
        if trivial:
            if x.is_cuda:
                y = F.dense_forward(x, kernel, epilogue=epilogue, sources2=x2, tuning=cfg.get("os_tuning"))
                if self._os_tuning_data is not None:
                    self._os_tuning_data.append((x.shape[0], x.shape[0], None, x, x2, None))
                epilogue_done = True
            else:
                y = torch.mm(x, kernel.view(self.in_channels, self.out_channels))
            coords, stride = inputs._coordinates, inputs._stride
        else:
            if self._kernel_map_cache is None:
                raise ValueError("Kernel map cache must be specified")
            skey = (inputs._stride, self.stride, self.transposed)
            stride = self._out_strides.get(skey)
            if stride is None:
                op = operator.floordiv if self.transposed else operator.mul
                stride = tuple(op(a, b) for a, b in zip(inputs._stride, self.stride))
                self._out_strides[skey] = stride
            cache = self._kernel_map_cache
            coords = cache.get_target_coordinates(inputs._coordinates, inputs._stride, stride, self.transposed)
            m = cache.get_kernel_map(inputs._coordinates, inputs._stride, coords, stride, self.kernel_size, d,
                                     force_os, self.transposed)
            # m = (S, T, map, t3, t4, t5, t6, mapsize, qmapsize) of the forward
            # (non-transposed) layer; a transposed layer swaps S and T
            S, T = (m[1], m[0]) if self.transposed else (m[0], m[1])
            if d == 0 or force_os:
                y = F.sparse_convolution_forward_os(S, T, m[2], x, kernel, epilogue=epilogue, sources2=x2,
                                                    tuning=cfg.get("os_tuning"))
                if self._os_tuning_data is not None:
                    mkey = (tuple(inputs._stride), tuple(stride), self.kernel_size)
                    if self.transposed:  # the transpose of the forward layer's map (its own row order)
                        mkey = ("transposed",) + mkey
                    self._os_tuning_data.append((S, T, m[2], x, x2, mkey))
            elif d == 1:
                y = F.sparse_convolution_forward_ws_merged(S, T, x, kernel, m[5], m[6], m[3], m[7], m[8],
                                                           self.transposed, epilogue=epilogue)
            elif d == 2:
                sm, tm = (m[4], m[3]) if self.transposed else (m[3], m[4])
                if self._tuning_data is not None:
                    self._tuning_data.append((sm, tm, m[5]))
                y = F.sparse_convolution_forward_ws(S, T, x, kernel, sm, tm, m[5], cfg["gather_tile_size"],
                                                    cfg["scatter_tile_size"], None, cfg["threshold"],
                                                    epilogue=epilogue)
            elif d % 2 == 1:
                dense = None if d == 3 else m[2]
                y = F.sparse_convolution_forward_hs_merged(S, T, x, kernel, m[5], m[6], m[3], dense, m[7],
                                                           m[8], self.transposed, epilogue=epilogue)
            else:
                sm, tm = (m[4], m[3]) if self.transposed else (m[3], m[4])
                dense = None if d == 4 else m[2]
                y = F.sparse_convolution_forward_hs(S, T, x, kernel, sm, tm, m[5], dense,
                                                    cfg["gather_tile_size"], cfg["scatter_tile_size"], None,
                                                    cfg["threshold"], epilogue=epilogue)
        if trivial and epilogue is not None and not epilogue_done:
            scale, shift, res, relu = epilogue
            y = y.float()
            if scale is not None:
                y = y * scale
            if shift is not None:
                y = y + shift
            if res is not None:
                y = y + res.float()
            if relu:
                y = torch.relu(y)
            y = y.to(x.dtype)
        elif bias is not None and epilogue is None:
            y += bias
        return SparseTensor(features=y, coordinates=coords, stride=stride)


def os_candidates(c_in: int, c_out: int, volume: int) -> List[List[int]]:
    """Values tried per output-stationary launch field (0 = automatic):
    column tiles up to the output width, step channels up to the padded input
    width, offset splits, offset packing where it applies (16-, 32- and
    64-channel inputs of kernels above 27 offsets), the block order (dispatch
    order, one range per XCD, or runs of 4 / 8 / 16 blocks per XCD), and the
    row walk (inputs of at most 16 channels with a map), the work balance
    (a row tile of a row-ordered map with more valid offsets than a third or
    a half of the kernel's split over blocks), and the cap on resident
    blocks per CU (the library's rule, none, one or two)."""
    cin_p = (c_in + 15) // 16 * 16
    cols = [0] + [c for c in (32, 64, 96, 128) if c <= (c_out + 31) // 32 * 32]
    steps = [0, 32] + ([64] if cin_p >= 64 else []) + ([128] if cin_p >= 96 else [])
    splits = [0, 1, 2, 4] if volume > 1 else [0]
    packs = [0, 1, 2, 4] if (volume > 27 and cin_p in (16, 32, 64)) else [0]
    walks = [0, 1] if (c_in <= 16 and volume > 1) else [0]
    balance = [0, (volume + 2) // 3, (volume + 1) // 2] if volume >= 8 else [0]
    return [cols, steps, splits, packs, [0, 1, 2, 3, 4], walks, balance, [0, -1, 1, 2]]


def time_os_calls(layer: "SparseConv", calls, tuning: tuple, reps: int) -> float:
    """Kernel time (ms) of a layer's recorded output-stationary calls under
    `tuning`; one call per distinct shape is timed."""
    from .functional import _native
    seen, total = set(), 0.0
    for S, T, omap, x, x2, _ in calls:
        key = (S, T, None if omap is None else omap.data_ptr(), x.shape[1], None if x2 is None else x2.shape[1])
        if key in seen:
            continue
        seen.add(key)
        total += _native._C.time_conv_os(S, T, omap, x, layer.kernel, reps, x2, tuple(tuning))
    return total


#: relative gain a launch choice must bring to replace the current one
OS_TUNING_MARGIN = 0.01


def choose_os_tuning(layer: "SparseConv", calls, reps: int = 10, row_order: Optional[int] = None,
                     with_time: bool = False):
    """Search over the launch fields of ``os_candidates``, twice over: the
    column tile and step channels as a pair over their whole grid, then each
    field in turn takes its fastest value with the others fixed; a value the
    library rejects is skipped.  The row-order field is
    held at `row_order` (default: the layer's current one, else -1, the
    library's rule).  Returns the tuning (and its time with `with_time`)."""
    if row_order is None:
        cur = layer._tunable_config.get("os_tuning")
        row_order = -1 if cur is None else int(cur[5])
    cands = os_candidates(layer.in_channels, layer.out_channels, int(np.prod(layer.kernel_size)))
    best = [0] * len(cands)

    def full(fields):  # (launch fields, row order, row walk)
        return tuple(fields[:5]) + (row_order,) + tuple(fields[5:])

    def cost(fields):
        try:
            return time_os_calls(layer, calls, full(fields), reps)
        except RuntimeError:
            F.cuda_reset_error()
            return float("inf")

    best_t = cost(best)

    def pair_grid():
        # the column tile and the step channels jointly (their best pair is
        # often not reached one field at a time: a narrower tile pays only
        # with shorter steps, which need the deeper ring)
        nonlocal best, best_t
        for col in cands[0]:
            for step in cands[1]:
                if (col, step) == (best[0], best[1]):
                    continue
                trial = list(best)
                trial[0], trial[1] = col, step
                t = cost(trial)
                if t < (1.0 - OS_TUNING_MARGIN) * best_t:
                    best, best_t = trial, t

    def each_field():
        nonlocal best, best_t
        for i, values in enumerate(cands):
            for v in values:
                if v == best[i]:
                    continue
                trial = list(best)
                trial[i] = v
                t = cost(trial)
                if t < (1.0 - OS_TUNING_MARGIN) * best_t:  # noise-sized gains do not move the search
                    best, best_t = trial, t

    # pair grid, fields, pair grid again (with the block order and splits
    # now chosen), fields
    pair_grid()
    each_field()
    pair_grid()
    each_field()
    tuning = full(best)
    return (tuning, best_t) if with_time else tuning
