"""Helpers and the per-layer dataflow selector.

The selector mirrors ``spira.tune`` (reference: source/spira/utils/helpers.py:
388-618): layers are grouped by ``(effective input stride, kernel size,
stride)``; each group is timed over every candidate ``map_dataflow`` in
0..8 (``force_os`` also tried for 1-4); downsampling groups are restricted to
dataflows 0-2; the arg-min is applied to the group and the results are saved
with ``torch.save`` as ``{'name_to_group', 'best_configs', 'layer_configs'}``
under ``<save_dir>/<tune_tag>.pt`` so that existing cache files keep loading.
Which candidate wins is measured on the machine at hand; only the candidate
set, grouping rule and file format are fixed.
"""
from __future__ import annotations

import contextlib
import functools
import itertools
import os
import time
from collections import defaultdict
from typing import Dict, Iterable, List, Optional, Tuple, Union

import torch
from torch.nn import Module

from .typing import ScalarOrTuple

__all__ = ["as_tuple", "make_divisible", "set_kernel_map_cache", "tune", "StableTimeAccumulator",
           "DataflowConfig", "set_config_for_group", "measure_model_time", "tune_dataflows", "tune_gs",
           "tune_os", "tune_row_orders", "apply_tuned_configs", "save_tuning_results", "load_tuning_results"]


def set_kernel_map_cache(module: Module, cache) -> Module:
    """Attach one KernelMapCache to every SparseConv below `module`."""
    if hasattr(module, "set_kernel_map_cache"):
        module.set_kernel_map_cache(cache)
    for child in module.children():
        set_kernel_map_cache(child, cache=cache)
    return module


def as_tuple(value: ScalarOrTuple, *, size: int = 3, name: Optional[str] = None) -> tuple:
    # (the common case first: a tuple of the right size, as every per-layer
    # call passes, costs one type and length check)
    if type(value) is tuple and len(value) == size:
        return value
    if type(value) is int:
        return (value,) * size
    if not isinstance(value, Iterable):
        return tuple(value for _ in range(size))
    value = tuple(value)
    if len(value) != size:
        raise ValueError(f"{name or 'Value'} must be a scalar or a iterable of size {size} "
                         f"but found {len(value)} elements")
    return value


def make_divisible(x: float, divisor: int = 8) -> int:
    return int((x + divisor / 2) // divisor * divisor)


class StableTimeAccumulator:
    """Running mean of timings that ignores samples above 5x the mean so far
    (reference helpers.py:49-75)."""

    def __init__(self):
        self.trial_count = 0
        self.average_time = 0.0

    def add_measurement(self, measured_time: float) -> None:
        if measured_time <= 0:
            return
        if self.trial_count == 0:
            self.average_time, self.trial_count = measured_time, 1
        elif measured_time <= 5 * self.average_time:
            self.average_time = (self.trial_count * self.average_time + measured_time) / (self.trial_count + 1)
            self.trial_count += 1

    def get_time(self) -> float:
        return self.average_time

    def get_trial_count(self) -> int:
        return self.trial_count


class DataflowConfig:
    def __init__(self, map_dataflow: int, force_os: bool = False):
        self.map_dataflow = map_dataflow
        self.force_os = force_os

    def apply_to_layer(self, layer) -> None:
        layer._tunable_config["map_dataflow"] = self.map_dataflow
        layer._tunable_config["force_os"] = self.force_os

    def __repr__(self):
        return f"DataflowConfig(map_dataflow={self.map_dataflow}, force_os={self.force_os})"


def set_config_for_group(model: Module, group_layers: List[str], config: DataflowConfig) -> None:
    """Apply `config` to a group; with force_os only the first half of the
    group's layers (in group order) runs output-stationary (helpers.py:96-116)."""
    modules = dict(model.named_modules())
    n_force = len(group_layers) // 2
    for idx, name in enumerate(group_layers):
        module = modules.get(name)
        if module is None:
            continue
        module._tunable_config["map_dataflow"] = config.map_dataflow
        module._tunable_config["force_os"] = bool(config.force_os and idx < n_force)


def measure_model_time(model: Module, input_data, kernel_map_cache=None) -> float:
    """Wall time of one forward pass with an empty kernel-map cache."""
    if kernel_map_cache is not None:
        kernel_map_cache.reset()
        assert len(kernel_map_cache._kernel_maps_cache) == 0, "Kernel map cache was not properly reset"
    torch.cuda.synchronize()
    start = time.time()
    with torch.no_grad():
        model(input_data)
    torch.cuda.synchronize()
    return time.time() - start


def _sparse_conv_cls():
    from ..nn.conv import SparseConv
    return SparseConv


#: relative margin by which a map's row order must beat index order (the
#: order's sort and the layers' lost L2 locality are not worth a tie)
ROW_ORDER_MARGIN = 0.02

#: relative margin by which a dataflow other than the first candidate must
#: beat it to be chosen (a deviation from the reference, which takes the
#: minimum)
DATAFLOW_MARGIN = 0.03


def tune_dataflows(model: Module, data_loader: Iterable, group_to_name: Dict[Tuple, List[str]],
                   config_options: List[DataflowConfig], kernel_map_cache, n_samples: int = 10,
                   verbose: bool = True) -> Dict[Tuple, DataflowConfig]:
    SparseConv = _sparse_conv_cls()
    gs_params = {name: {k: m._tunable_config[k] for k in ("gather_tile_size", "scatter_tile_size", "threshold")}
                 for name, m in model.named_modules() if isinstance(m, SparseConv)}
    modules = dict(model.named_modules())

    def restore(names):
        for name in names:
            if name in gs_params:
                modules[name]._tunable_config.update(gs_params[name])

    best: Dict[Tuple, DataflowConfig] = {}
    for group_id, names in group_to_name.items():
        ksize, lstride = group_id[1], group_id[2]
        if all(s == 1 for s in lstride) and all(k == 1 for k in ksize):
            continue  # trivial 1x1 layers run torch.mm whatever the config
        if any(s > 1 for s in lstride):
            candidates = [c for c in config_options if c.map_dataflow in (0, 1, 2)]
        else:
            candidates = list(config_options)
        times = defaultdict(StableTimeAccumulator)
        for cfg in candidates:
            restore(names)
            set_config_for_group(model, names, cfg)
            for idx, sample in enumerate(data_loader):
                try:
                    elapsed = measure_model_time(model, sample, kernel_map_cache)
                except RuntimeError as e:  # a candidate that fails is never chosen
                    if verbose:
                        print(f"  {cfg} failed: {e}")
                    elapsed = None
                    break
                if idx > 2:
                    times[str(cfg)].add_measurement(elapsed)
                if idx + 1 >= n_samples:
                    break
            if verbose and str(cfg) in times:
                print(f"  {group_id} {cfg}: {times[str(cfg)].get_time() * 1e3:.3f} ms")
        measured = [c for c in candidates if times[str(c)].get_trial_count() > 0]
        if not measured:
            measured = candidates[:1]
        t_of = lambda c: times[str(c)].get_time() if times[str(c)].get_trial_count() else float("inf")
        pick = min(measured, key=t_of)
        # another dataflow than the first candidate (the output-stationary
        # one) must win by DATAFLOW_MARGIN: the timings are wall times of a
        # few forward passes whose maps are built layer by layer, and noise of
        # that size flipped groups to weight-stationary maps that cost more
        # inside a network-wide map build than here
        first = measured[0]
        if pick is not first and t_of(pick) > (1.0 - DATAFLOW_MARGIN) * t_of(first):
            pick = first
        best[group_id] = pick
        if verbose:
            print(f"  -> {group_id}: {best[group_id]}")
    for name, params in gs_params.items():
        modules[name]._tunable_config.update(params)
    return best


def tune_gs(model: Module, kernel_map_cache, data_loader, n_samples: int = 10) -> None:
    """Run samples with every SparseConv recording its gather/scatter masks,
    then let each layer sweep its bucket threshold and tile sizes."""
    SparseConv = _sparse_conv_cls()
    with contextlib.ExitStack() as stack:
        for m in model.modules():
            if isinstance(m, SparseConv):
                stack.enter_context(m.tune_gs())
        for i, sample in enumerate(data_loader):
            kernel_map_cache.reset()
            model(sample)
            if i + 1 >= n_samples:
                break


def _forward_once(model: Module, kernel_map_cache, sample) -> None:
    if kernel_map_cache is not None:
        kernel_map_cache.reset()
    with torch.no_grad():
        model(sample)
    torch.cuda.synchronize()


def tune_os(model: Module, kernel_map_cache, sample, reps: int = 10, verbose: bool = False) -> None:
    """Output-stationary launch choices of every fp16 layer that runs the
    output-stationary kernel (``SparseConv.tune_os``), from one forward pass
    of `sample`, then the row order per map (``tune_row_orders``)."""
    SparseConv = _sparse_conv_cls()
    with contextlib.ExitStack() as stack:
        for m in model.modules():
            if isinstance(m, SparseConv):
                stack.enter_context(m.tune_os(reps))
        _forward_once(model, kernel_map_cache, sample)
    tune_row_orders(model, kernel_map_cache, sample, reps, verbose)


def _row_order_ms(omap: torch.Tensor, num_targets: int, reps: int = 5) -> float:
    """GPU time (ms) to compute a map's row order (on fresh copies: the order
    is cached per map tensor).  The calls are queued behind a short GPU wait,
    so that the host's work per call (allocations, launches) overlaps the
    GPU as it does inside a network's map build, and only device time is
    counted."""
    from ..nn.functional import _native
    copies = [omap.clone() for _ in range(reps)]
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda._sleep(2_000_000)  # ~1 ms of GPU clock cycles: longer than the host's queueing
    a.record()
    for c in copies:
        _native._C.kmap_row_order(c, int(num_targets))
    b.record()
    b.synchronize()
    return a.elapsed_time(b) / reps


def _share_sibling_tunings(entries, picks, reps: int) -> None:
    """Layers of the same shape on the same map (a res block's repeated
    convolutions) are the same launch problem: each also tries the tunings
    its siblings found, and keeps the fastest (the searches start from the
    same point, but timing noise can send them to different optima)."""
    from ..nn.conv import time_os_calls, OS_TUNING_MARGIN
    for i, (m, call) in enumerate(entries):
        for j, (m2, _) in enumerate(entries):
            if j == i or (m2.in_channels, m2.out_channels, m2.kernel.shape) != (m.in_channels, m.out_channels,
                                                                                 m.kernel.shape):
                continue
            if picks[j][0] == picks[i][0]:
                continue
            try:
                t = time_os_calls(m, [call], picks[j][0], reps)
            except RuntimeError:  # a launch this layer cannot take
                from ..nn import functional as F
                F.cuda_reset_error()
                continue
            if t < (1.0 - OS_TUNING_MARGIN) * picks[i][1]:
                picks[i] = (picks[j][0], t)


def tune_row_orders(model: Module, kernel_map_cache, sample, reps: int = 10,
                    verbose: bool = False) -> Dict[Tuple, int]:
    """Walk each output-stationary map (8..128 offsets; a transposed layer's
    map is a map of its own) in row order or not, whichever is faster for
    the layers that read it, counting the order's sort once per map.  The
    launch choices depend on
    the order (a row-ordered walk skips more offsets and prefers other step
    and tile sizes), so each layer's launch is searched again under both
    orders.  Sets every such layer's tuning and the cache's request for the
    map; returns the requests."""
    SparseConv = _sparse_conv_cls()
    from ..nn.conv import choose_os_tuning
    convs = [m for m in model.modules() if isinstance(m, SparseConv)]
    for m in convs:
        m._os_tuning_data = []
    try:
        _forward_once(model, kernel_map_cache, sample)
        by_map: Dict[Tuple, list] = defaultdict(list)
        for m in convs:
            if m.kernel.dtype != torch.float16 or not m.kernel.is_cuda:
                continue
            for call in m._os_tuning_data:
                omap, key = call[2], call[5]
                if omap is None or key is None or not (8 <= omap.shape[1] <= 128):
                    continue
                by_map[key].append((m, call))
        requests: Dict[Tuple, int] = {}
        for key, entries in by_map.items():
            totals, picks = {}, {}
            for r in (0, 1):
                picks[r] = [choose_os_tuning(m, [call], reps, row_order=r, with_time=True) for m, call in entries]
                _share_sibling_tunings(entries, picks[r], reps)
                totals[r] = sum(t for _, t in picks[r])
            omap, T = entries[0][1][2], entries[0][1][1]
            # with the order computed, each layer still walks whichever is
            # faster for it: the map's order pays if the layers' best walks
            # plus the sort beat index order everywhere
            best1 = [min(t0, t1) for (_, t0), (_, t1) in zip(picks[0], picks[1])]
            # (an order made with the map, as a transposed layer's
            # partition inverse carries one, costs no sort)
            from ..nn.functional import _native
            sort_ms = 0.0 if _native._C.has_free_row_order(omap, int(T)) else _row_order_ms(omap, T)
            totals[1] = sum(best1) + sort_ms
            r = 1 if totals[1] < (1.0 - ROW_ORDER_MARGIN) * totals[0] else 0
            requests[key] = r
            if verbose:
                print(f"[Spira] map {key}: {len(entries)} layers, {1e3 * totals[0]:.1f} us in index order, "
                      f"{1e3 * totals[1]:.1f} us with the order (each layer its faster walk, sort included) -> row order {r}")
                for (m, _), (t0, ms0), (t1, ms1) in zip(entries, picks[0], picks[1]):
                    print(f"    {m.in_channels}->{m.out_channels}: {t0} {1e3 * ms0:.1f} us | {t1} {1e3 * ms1:.1f} us")
            for (m, _), (tn0, t0), (tn1, t1) in zip(entries, picks[0], picks[1]):
                m._tunable_config["os_tuning"] = tn1 if (r == 1 and t1 < t0) else tn0
        if kernel_map_cache is not None:
            kernel_map_cache.row_order_requests.update(requests)
        return requests
    finally:
        for m in convs:
            m._os_tuning_data = None


def apply_tuned_configs(model: Module, name_to_group: Dict[str, Tuple], best_configs: Dict[Tuple, DataflowConfig],
                        layer_configs: Optional[Dict[str, Dict]] = None) -> None:
    SparseConv = _sparse_conv_cls()
    if layer_configs:
        for name, m in model.named_modules():
            if isinstance(m, SparseConv) and name in layer_configs:
                cfg = layer_configs[name]
                for k in ("gather_tile_size", "scatter_tile_size", "threshold", "os_tuning"):
                    if k in cfg:
                        m._tunable_config[k] = tuple(cfg[k]) if k == "os_tuning" and cfg[k] is not None \
                            else cfg[k]
    group_to_layers = defaultdict(list)
    for name, gid in name_to_group.items():
        group_to_layers[gid].append(name)
    for gid, layers in group_to_layers.items():
        if gid in best_configs:
            set_config_for_group(model, layers, best_configs[gid])


def save_tuning_results(name_to_group: Dict, best_configs: Dict[Tuple, DataflowConfig], save_path: str,
                        model: Module, row_order_requests: Optional[Dict[Tuple, int]] = None) -> None:
    SparseConv = _sparse_conv_cls()
    d = os.path.dirname(save_path)
    if d:
        os.makedirs(d, exist_ok=True)
    layer_configs = {name: dict(m._tunable_config) for name, m in model.named_modules()
                     if isinstance(m, SparseConv)}
    torch.save({
        "name_to_group": name_to_group,
        "best_configs": {k: {"map_dataflow": v.map_dataflow, "force_os": v.force_os}
                         for k, v in best_configs.items()},
        "layer_configs": layer_configs,
        "row_order_requests": dict(row_order_requests or {}),
    }, save_path)


def load_tuning_results(load_path: str, with_row_orders: bool = False):
    # the file holds only dicts / tuples / numbers: the weights-only loader suffices
    data = torch.load(load_path, weights_only=True)
    best = {k: DataflowConfig(v["map_dataflow"], v["force_os"]) for k, v in data["best_configs"].items()}
    if with_row_orders:
        return data["name_to_group"], best, data.get("layer_configs", {}), data.get("row_order_requests", {})
    return data["name_to_group"], best, data.get("layer_configs", {})


def tune(model: Module, data_loader: Iterable, kernel_map_cache=None, map_dataflow_options: List[int] = None,
         test_force_os: bool = True, n_samples: int = 10, n_samples_for_gs: int = 1,
         save_dir: str = ".tune_configs", tune_tag: str = "default", force_retune: bool = False,
         allow_gs_tuning: bool = True, verbose: bool = False,
         return_dataflows: bool = False, allow_os_tuning: bool = True) -> Union[Module, Tuple[Module, Dict]]:
    """Select a dataflow per layer group by measurement (see module doc),
    then (``allow_os_tuning``) the output-stationary launch choices of every
    layer and the row order of every output-stationary map."""
    SparseConv = _sparse_conv_cls()
    if map_dataflow_options is None:
        map_dataflow_options = list(range(9))
    samples = list(itertools.islice(data_loader, n_samples + 1))
    options: List[DataflowConfig] = []
    for d in map_dataflow_options:
        options.append(DataflowConfig(d, False))
        if test_force_os and d in (1, 2, 3, 4):
            options.append(DataflowConfig(d, True))

    save_path = os.path.join(save_dir, f"{tune_tag}.pt")
    if os.path.exists(save_path) and not force_retune:
        try:
            name_to_group, best, layer_configs, requests = load_tuning_results(save_path, with_row_orders=True)
            apply_tuned_configs(model, name_to_group, best, layer_configs)
            if kernel_map_cache is not None:
                kernel_map_cache.row_order_requests.update(requests)
            groups = {g: c.map_dataflow for g, c in best.items()}
            return (model, groups) if return_dataflows else model
        except Exception as e:  # unreadable cache: tune again
            if verbose:
                print(f"Warning: Could not load cache ({e}). Re-tuning...")

    if allow_gs_tuning:
        tune_gs(model, kernel_map_cache, samples, n_samples=n_samples_for_gs)

    name_to_group: Dict[str, Tuple] = {}
    group_to_name: Dict[Tuple, List[str]] = defaultdict(list)

    def hook(module, inputs, outputs, name):
        stride = inputs[0]._stride
        eff = tuple(stride[k] // module.stride[k] for k in range(3)) if module.transposed else stride
        gid = (eff, module.kernel_size, module.stride)
        name_to_group[name] = gid
        group_to_name[gid].append(name)

    handles = [m.register_forward_hook(functools.partial(hook, name=n))
               for n, m in model.named_modules() if isinstance(m, SparseConv)]
    try:
        if samples:
            if kernel_map_cache is not None:
                kernel_map_cache.reset()
            with torch.no_grad():
                model(samples[0])
    finally:
        for h in handles:
            h.remove()

    best = tune_dataflows(model, samples, group_to_name, options, kernel_map_cache, n_samples=n_samples,
                          verbose=verbose)
    apply_tuned_configs(model, name_to_group, best, None)
    requests: Dict[Tuple, int] = {}
    if allow_os_tuning and samples and torch.cuda.is_available():
        tune_os(model, kernel_map_cache, samples[0], verbose=verbose)
        if kernel_map_cache is not None:
            requests = dict(kernel_map_cache.row_order_requests)
    save_tuning_results(name_to_group, best, save_path, model, requests)
    groups = {g: c.map_dataflow for g, c in best.items()}
    return (model, groups) if return_dataflows else model
