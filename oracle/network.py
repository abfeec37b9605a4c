"""Whole-network forward pass on the CPU through the oracle.

TEST INFRASTRUCTURE ONLY: used by tests/ (network-level parity of the GPU
path) and by ``bench.py``'s ``cpu_baseline`` leg (the reference-semantics CPU
timing), always as the checker; the product path never imports it.

It evaluates a spira_amd network module by module in fp32 with the oracle's
maps (output-stationary layout, torch/cuda_sparse_convolution_mapping.cu:
211-892) and convolutions (``conv_os_f32``), eval-mode batch norm, ReLU, the
residual blocks and the UNet's skip concatenations (models/unet.py of the
reference: channel concatenation [upsampled, skip]), so that it follows the
same module graph as the GPU forward.  Layer semantics are the ones pinned
in tests/test_oracle.py; the network composition itself is plain numpy.
"""
from __future__ import annotations

from typing import Dict, List, Tuple

import numpy as np

from . import oracle as orc

Stride = Tuple[int, int, int]


def network_forward(model, coords_np: np.ndarray, feats_np: np.ndarray,
                    dataflow="layer") -> List[Tuple[np.ndarray, Stride]]:
    """Outputs of ``model`` (SparseResUNet42-style: ``stem`` / ``encoders`` /
    ``decoders``; or a SparseResNet-style ModuleList of stages) as
    (features in sorted-key order, tensor stride) pairs, like the GPU
    forward's SparseTensors after ``order()``.

    ``dataflow`` is the map dataflow every layer runs on, with that
    dataflow's semantics: 0 -- the output-stationary map and z-major weight
    rows (convert_weights.py:19-28); 1 -- the compacted pair lists with the
    mirrored half map of submanifold layers (weight_stat.cuh semantics,
    sparse_convolution.cu:1267-1295); 2 -- the gather / scatter masks with
    their half map (sparse_convolution.cu:1002-1124).  Dataflows 1 and 2 use
    canonical weight rows.  The half maps differ from the full map where the
    reference's z walk wraps (voxels at x = y = 0), so each dataflow is
    evaluated with its own maps.  ``"layer"`` (the default): each layer's own
    ``_tunable_config["map_dataflow"]`` (0, 1 or 2; what the selector chose
    for its group)."""
    import torch
    from spira_amd import nn as spnn
    from spira_amd.networks import SparseResBlock

    if dataflow not in (0, 1, 2, "layer"):
        raise ValueError(f"dataflow must be 0, 1, 2 or 'layer', not {dataflow}")
    keys, perm = orc.flatten_sort(coords_np, True)
    x = np.ascontiguousarray(feats_np[perm], dtype=np.float32)
    vox: Dict[Stride, np.ndarray] = {(1, 1, 1): keys}
    maps: Dict[tuple, tuple] = {}

    def coords_of(stride):
        if stride not in vox:
            vox[stride] = orc.downsample(keys, stride)
        return vox[stride]

    def conv(layer, feats, stride):
        W = layer.kernel.detach().float().cpu().numpy()
        d = layer._tunable_config["map_dataflow"] if dataflow == "layer" else dataflow
        if d not in (0, 1, 2) or layer._tunable_config.get("force_os", False):
            raise ValueError(f"the oracle network evaluates dataflows 0, 1 and 2 without force_os, not {d}")
        if layer.is_trivial:
            return feats @ W[0], stride
        if layer.transposed:
            out_stride = tuple(a // b for a, b in zip(stride, layer.stride))
            key = (out_stride, stride, layer.kernel_size)
        else:
            out_stride = tuple(a * b for a, b in zip(stride, layer.stride))
            key = (stride, out_stride, layer.kernel_size)
        key = key + (d,)
        if key not in maps:
            maps[key] = orc.build_kmap(coords_of(key[0]), coords_of(key[1]), layer.kernel_size, key[0], d)
        m = maps[key]
        S, T = (m[1], m[0]) if layer.transposed else (m[0], m[1])
        if d == 0:
            omap = orc.convert_transposed_os(m[2], m[0]) if layer.transposed else m[2]
            return orc.conv_os_f32(omap, T, feats, W), out_stride
        if d == 1:
            y = orc.conv_ws_merged(S, T, feats, W, m[5], m[3], transpose=layer.transposed)
        else:
            sm, tm = (m[4], m[3]) if layer.transposed else (m[3], m[4])
            y = orc.conv_ws_gs(S, T, feats, W, sm, tm)
        return y.astype(np.float32), out_stride

    def run(mod, feats, stride):
        if isinstance(mod, spnn.SparseConv):
            return conv(mod, feats, stride)
        if isinstance(mod, spnn.BatchNorm):
            rm, rv = mod.running_mean.float().cpu().numpy(), mod.running_var.float().cpu().numpy()
            g, b = mod.weight.detach().float().cpu().numpy(), mod.bias.detach().float().cpu().numpy()
            return (feats - rm) / np.sqrt(rv + mod.eps) * g + b, stride
        if isinstance(mod, spnn.ReLU):
            return np.maximum(feats, 0), stride
        if isinstance(mod, torch.nn.Identity):
            return feats, stride
        if isinstance(mod, SparseResBlock):
            a, s1 = run(mod.main, feats, stride)
            b, _ = run(mod.shortcut, feats, stride)
            return np.maximum(a + b, 0), s1
        if isinstance(mod, torch.nn.Sequential):
            for sub in mod:
                feats, stride = run(sub, feats, stride)
            return feats, stride
        raise TypeError(type(mod))

    def level(feats, stride, encoders, decoders):
        if len(encoders) == 0:
            return [(feats, stride)]
        f2, s2 = run(encoders[0], feats, stride)
        outs = level(f2, s2, encoders[1:], decoders[:-1])
        up, su = run(decoders[-1]["upsample"], *outs[-1])
        y, sy = run(decoders[-1]["fuse"], np.concatenate([up, feats], axis=1), su)
        return [(feats, stride)] + outs + [(y, sy)]

    if hasattr(model, "stem"):
        f, s = run(model.stem, x, (1, 1, 1))
        return level(f, s, list(model.encoders), list(model.decoders))
    outs = []
    f, s = x, (1, 1, 1)
    for stage in model:
        f, s = run(stage, f, s)
        outs.append((f, s))
    return outs
