"""Epilogue fusion for inference: batch norm (eval mode), ReLU and the
residual add of a res block are folded into the output write of the
preceding SparseConv, so that a conv + BN + ReLU (+ residual) chain costs
one kernel instead of four element-wise passes over the features.

No reference counterpart: the reference runs batch norm, ReLU and the
residual add as separate ops (scripts/models/spira/modules/blocks.py:12-84,
source/spira/nn/normalizations.py:8-10, activations.py:8-18).

`fuse_epilogues(model)` only annotates modules; the model's structure,
parameters and state_dict keys are unchanged.  A fused chain takes the
fused path when it is numerically the same op: autograd off and the batch
norm in eval mode (running statistics).  Otherwise every module runs as
written.
"""
from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import nn

__all__ = ["fuse_epilogues", "bn_affine"]


def bn_affine(bn: nn.BatchNorm1d) -> Tuple[torch.Tensor, torch.Tensor]:
    """(scale, shift) fp32 of an eval-mode batch norm, cached while its
    parameters and running statistics are unchanged:
    scale = weight / sqrt(running_var + eps), shift = bias - running_mean * scale."""
    # (the module's dicts read directly: this runs once per fused layer and step)
    p, b = bn._parameters, bn._buffers
    w, bb, rm, rv = p.get("weight"), p.get("bias"), b.get("running_mean"), b.get("running_var")
    key = (-1 if w is None else w._version, -1 if bb is None else bb._version,
           -1 if rm is None else rm._version, -1 if rv is None else rv._version)
    cached = bn.__dict__.get("_spira_affine")
    if cached is not None and cached[0] == key and cached[1].device == rm.device:
        return cached[1], cached[2]
    with torch.no_grad():
        inv = torch.rsqrt(bn.running_var.float() + bn.eps)
        scale = inv * bn.weight.float() if bn.weight is not None else inv
        shift = -bn.running_mean.float() * scale
        if bn.bias is not None:
            shift = shift + bn.bias.float()
        scale, shift = scale.contiguous(), shift.contiguous()
    object.__setattr__(bn, "_spira_affine", (key, scale, shift))
    return scale, shift


def _absorb(mod: nn.Module, conv: nn.Module) -> None:
    # a plain attribute (not a registered submodule): state_dict is unchanged
    object.__setattr__(mod, "_spira_absorbed_by", conv)


def absorbed(mod: nn.Module) -> bool:
    """True when `mod` (a batch norm / ReLU) is applied by a fused conv."""
    conv = mod.__dict__.get("_spira_absorbed_by")  # (set with object.__setattr__)
    return conv is not None and conv._fused_active()


def _fuse_sequential(seq: nn.Sequential) -> None:
    from .activations import ReLU
    from .conv import SparseConv
    from .normalizations import BatchNorm
    mods = list(seq.children())
    i = 0
    while i < len(mods):
        conv = mods[i]
        if not isinstance(conv, SparseConv) or conv._epi_bn is not None or conv._epi_relu:
            i += 1
            continue
        j = i + 1
        if j < len(mods) and type(mods[j]) is BatchNorm and mods[j].track_running_stats:
            object.__setattr__(conv, "_epi_bn", mods[j])
            _absorb(mods[j], conv)
            j += 1
        if j < len(mods) and type(mods[j]) is ReLU:
            conv._epi_relu = True
            _absorb(mods[j], conv)
            j += 1
        i = j


def fuse_epilogues(model: nn.Module) -> nn.Module:
    """Annotate `model` so that SparseConv -> BatchNorm -> ReLU chains inside
    nn.Sequential containers, and the residual add + ReLU of SparseResBlock,
    run as one fused conv at inference.  Returns the model."""
    from ..networks import SparseResBlock
    for m in model.modules():
        if isinstance(m, nn.Sequential):
            _fuse_sequential(m)
    for m in model.modules():
        if isinstance(m, SparseResBlock):
            last = m.main[3]
            if last._epi_relu:
                continue
            last._epi_relu = True
            _absorb(m.relu, last)
            m._fused = True
    return model
