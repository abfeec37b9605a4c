"""Benchmark networks built from the spira API: the MinkUNet-style
SparseResUNet42 and the SparseResNet backbones that the reference's
experiments run (reference: scripts/models/spira/sparse_unet.py:14-119,
sparse_resnet.py:12-85, modules/blocks.py:12-84), plus their network-wide
kernel-map schedules (scripts/end_to_end_experiment.py:93-112).

The layer structure is fixed by the reference models (same channel counts,
kernel sizes and strides) so that checkpoints and tuned configs line up.
"""
from __future__ import annotations

from typing import List, Tuple, Union

import numpy as np
from torch import nn

from . import nn as spnn
from .nn.fusion import absorbed
from .operators import cat
from .tensors import SparseTensor

__all__ = ["SparseConvBlock", "SparseConvTransposeBlock", "SparseResBlock", "SparseResUNet42", "SparseResNet21D",
           "SparseResNetLarge", "kmap_schedule"]

IntOrTuple = Union[int, Tuple[int, ...], List[int]]


class _Chain(nn.Sequential):
    """nn.Sequential that does not call the batch norms and ReLUs a fused
    convolution applies (they would return their input unchanged): the
    per-module call costs host time that a small layer's kernel does not
    cover.  Same children and state_dict keys as nn.Sequential."""

    def forward(self, x):
        for m in self:
            if not absorbed(m):
                x = m(x)
        return x


class SparseConvBlock(_Chain):
    def __init__(self, cin: int, cout: int, kernel_size: IntOrTuple, stride: IntOrTuple = 1):
        super().__init__(spnn.SparseConv(cin, cout, kernel_size, stride=stride), spnn.BatchNorm(cout),
                         spnn.ReLU(True))


class SparseConvTransposeBlock(_Chain):
    def __init__(self, cin: int, cout: int, kernel_size: IntOrTuple, stride: IntOrTuple = 1):
        super().__init__(spnn.SparseConv(cin, cout, kernel_size, stride=stride, transposed=True),
                         spnn.BatchNorm(cout), spnn.ReLU(True))


class SparseResBlock(nn.Module):
    def __init__(self, cin: int, cout: int, kernel_size: IntOrTuple, stride: IntOrTuple = 1):
        super().__init__()
        self.main = _Chain(
            spnn.SparseConv(cin, cout, kernel_size, stride=stride), spnn.BatchNorm(cout), spnn.ReLU(True),
            spnn.SparseConv(cout, cout, kernel_size), spnn.BatchNorm(cout))
        if cin != cout or np.prod(stride) != 1:
            self.shortcut = _Chain(spnn.SparseConv(cin, cout, 1, stride=stride), spnn.BatchNorm(cout))
        else:
            self.shortcut = nn.Identity()
        self.relu = spnn.ReLU(True)
        self._fused = False  # set by spira_amd.nn.fuse_epilogues

    def forward(self, x: SparseTensor) -> SparseTensor:
        if self._fused:
            c0, n0, r0, c1, n1 = self.main
            if c1._fused_active():
                # the shortcut's output is the residual of the second conv's epilogue
                sc = self.shortcut(x)
                h = c0(x)
                if not absorbed(n0):
                    h = n0(h)
                if not absorbed(r0):
                    h = r0(h)
                h = c1(h, residual=sc)
                return h if absorbed(n1) else n1(h)
        return self.relu(self.main(x) + self.shortcut(x))


class _SparseResUNet(nn.Module):
    def __init__(self, stem_channels: int, encoder_channels: List[int], decoder_channels: List[int], *,
                 in_channels: int = 4, width_multiplier: float = 1.0):
        super().__init__()
        ch = [int(width_multiplier * c) for c in [stem_channels] + encoder_channels + decoder_channels]
        self.stem = _Chain(
            spnn.SparseConv(in_channels, ch[0], 3), spnn.BatchNorm(ch[0]), spnn.ReLU(True),
            spnn.SparseConv(ch[0], ch[0], 3), spnn.BatchNorm(ch[0]), spnn.ReLU(True))
        self.encoders = nn.ModuleList(
            nn.Sequential(SparseConvBlock(ch[k], ch[k], 2, stride=2), SparseResBlock(ch[k], ch[k + 1], 3),
                          SparseResBlock(ch[k + 1], ch[k + 1], 3))
            for k in range(4))
        self.decoders = nn.ModuleList(
            nn.ModuleDict({
                "upsample": SparseConvTransposeBlock(ch[k + 4], ch[k + 5], 2, stride=2),
                "fuse": nn.Sequential(SparseResBlock(ch[k + 5] + ch[3 - k], ch[k + 5], 3),
                                      SparseResBlock(ch[k + 5], ch[k + 5], 3)),
            })
            for k in range(4))

    def _level(self, x: SparseTensor, k: int) -> List[SparseTensor]:
        """Encoder level k and everything below it; decoder n - 1 - k joins
        its output with x (module lists indexed, not sliced: a slice builds
        a new ModuleList on every call)."""
        n = len(self.encoders)
        if k == n:
            return [x]
        outputs = self._level(self.encoders[k](x), k + 1)
        dec = self.decoders[n - 1 - k]
        up = dec["upsample"](outputs[-1])
        y = dec["fuse"](cat([up, x]))
        return [x] + outputs + [y]

    def forward(self, x: SparseTensor) -> List[SparseTensor]:
        return self._level(self.stem(x), 0)


class SparseResUNet42(_SparseResUNet):
    def __init__(self, **kwargs):
        super().__init__(32, [32, 64, 128, 256], [256, 128, 96, 96], **kwargs)


class _SparseResNet(nn.ModuleList):
    def __init__(self, blocks, *, in_channels: int = 4, width_multiplier: float = 1.0):
        super().__init__()
        for num_blocks, cout, ksize, stride in blocks:
            cout = int(cout * width_multiplier)
            mods = []
            for i in range(num_blocks):
                if i == 0:
                    mods.append(SparseConvBlock(in_channels, cout, ksize, stride=stride))
                else:
                    mods.append(SparseResBlock(in_channels, cout, ksize))
                in_channels = cout
            self.append(nn.Sequential(*mods))

    def forward(self, x: SparseTensor) -> List[SparseTensor]:
        outs = []
        for m in self:
            x = m(x)
            outs.append(x)
        return outs


class SparseResNet21D(_SparseResNet):
    def __init__(self, **kwargs):
        super().__init__([(3, 16, 3, 1), (3, 32, 3, 2), (3, 64, 3, 2), (3, 128, 3, 2),
                          (1, 128, (1, 1, 3), (1, 1, 2))], **kwargs)


class SparseResNetLarge(_SparseResNet):
    def __init__(self, **kwargs):
        super().__init__([(3, 16, 5, 1), (3, 32, 5, 2), (3, 64, 5, 2), (3, 128, 5, 2)], **kwargs)


def kmap_schedule(model: str):
    """(target_strides, kernel_sizes, source_strides) for
    KernelMapCache.add_all_kernel_maps: map i goes from source_strides[i] to
    source_strides[i+1] with kernel_sizes[i] (end_to_end_experiment.py:93-112)."""
    if model == "UNet":
        ts = [(2, 2, 2), (4, 4, 4), (8, 8, 8), (16, 16, 16)]
        ks = [(3, 3, 3), (2, 2, 2)] * 4 + [(3, 3, 3)]
        ss = [(1, 1, 1), (1, 1, 1), (2, 2, 2), (2, 2, 2), (4, 4, 4), (4, 4, 4), (8, 8, 8), (8, 8, 8),
              (16, 16, 16), (16, 16, 16)]
    elif model == "ResNetLarge":
        ts = [(2, 2, 2), (4, 4, 4), (8, 8, 8)]
        ks = [(5, 5, 5)] * 7
        ss = [(1, 1, 1), (1, 1, 1), (2, 2, 2), (2, 2, 2), (4, 4, 4), (4, 4, 4), (8, 8, 8), (8, 8, 8)]
    elif model == "ResNet":
        ts = [(2, 2, 2), (4, 4, 4), (8, 8, 8), (8, 8, 16)]
        ks = [(3, 3, 3)] * 7 + [(1, 1, 3)]
        ss = [(1, 1, 1), (1, 1, 1), (2, 2, 2), (2, 2, 2), (4, 4, 4), (4, 4, 4), (8, 8, 8), (8, 8, 8), (8, 8, 16)]
    else:
        raise ValueError(model)
    return ts, ks, ss
