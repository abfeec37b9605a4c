"""Whole networks on the GPU against the oracle (oracle/network.py: the same
module graph evaluated in fp32 with the oracle's maps and convolutions):
SparseResUNet42 (config 4's network; k = 3 and k = 2 maps, transposed
layers, skip concatenations) and SparseResNetLarge (config 5's network;
k = 5, 125-offset maps, stride-2 k = 5 transitions), both fp16 with fused
epilogues and the network-wide map build of KernelMapCache.  Every output
of every level: coordinates bit-exact, features within
max |error| <= 1e-2 * RMS(reference), the north star's fp16 bound, although
fp16 activations are rounded again after every one of the ~20-40 layers in
between."""
import numpy as np
import pytest
import torch

import spira_amd
from oracle import oracle as orc
from oracle.network import network_forward
from spira_amd import scenes
from spira_amd.networks import SparseResNetLarge, SparseResUNet42, kmap_schedule

from helpers import np_, rel_err

pytestmark = pytest.mark.gpu

NET_TOL = 1e-2


def _randomise_norms(model, seed):
    g = torch.Generator().manual_seed(seed)
    for m in model.modules():
        if isinstance(m, spira_amd.nn.BatchNorm):
            n = m.running_mean.numel()
            m.running_mean.copy_(0.1 * torch.randn(n, generator=g))
            m.running_var.copy_(0.5 + torch.rand(n, generator=g))
            m.weight.data.copy_(0.5 + torch.rand(n, generator=g))
            m.bias.data.copy_(0.1 * torch.randn(n, generator=g))


def _gpu_forward(model, schedule, coords, feats, dev):
    # every layer on the output-stationary dataflow, the maps built for it
    for m in model.modules():
        if isinstance(m, spira_amd.nn.SparseConv):
            m._tunable_config["map_dataflow"] = 0
    cache = spira_amd.nn.KernelMapCache()
    spira_amd.set_kernel_map_cache(model, cache)
    ts, ks, ss = kmap_schedule(schedule)
    x = spira_amd.SparseTensor(coordinates=torch.from_numpy(coords).to(dev),
                               features=torch.from_numpy(feats).to(dev).half(), double=True)
    x.order()
    cache.add_all_kernel_maps(x._coordinates, ks, ss, ts, (1, 1, 1), [0] * len(ks))
    with torch.no_grad():
        return model(x)


@pytest.mark.parametrize("name", ["UNet", "ResNetLarge"])
def test_network_matches_oracle(dev, name):
    if name == "UNet":
        coords = scenes.spheres_planes(n=20_000, grid=128, seed=21)
        model, cin = SparseResUNet42(in_channels=3), 3
    else:
        coords = scenes.lidar_blobs(target=20_000, seed=22)
        model, cin = SparseResNetLarge(in_channels=4), 4
    torch.manual_seed(5)
    _randomise_norms(model, 6)
    model = model.eval()
    feats = np.random.default_rng(7).standard_normal((len(coords), cin)).astype(np.float32)
    # oracle first, on the fp32 weights rounded to fp16 (the GPU network's weights)
    model = model.half().float()
    ref = network_forward(model, coords, feats, 0)
    gpu_model = model.to(dev).half().eval()
    spira_amd.nn.fuse_epilogues(gpu_model)
    out = _gpu_forward(gpu_model, name, coords, feats, dev)
    assert len(out) == len(ref)
    rk, _ = orc.flatten_sort(coords, True)
    for i, (o, (rf, rs)) in enumerate(zip(out, ref)):
        assert tuple(o.stride) == tuple(rs), f"output {i}: stride {o.stride} != {rs}"
        want = rk if tuple(rs) == (1, 1, 1) else orc.downsample(rk, tuple(rs))
        assert np.array_equal(np_(o.coordinates), want), f"output {i}: coordinates differ"
        assert o.features.shape == rf.shape, f"output {i}: shape {tuple(o.features.shape)} != {rf.shape}"
        err = rel_err(np_(o.features.float()), rf)
        print(f"{name} output {i} stride {tuple(rs)}: max |error| = {err:.3g} x RMS", flush=True)
        assert err <= NET_TOL, f"{name} output {i} (stride {rs}): error {err:.3g} x RMS"


def test_repeated_steps_keep_memory_flat(dev):
    """Many inference steps in one process, each with a fresh map cache (the
    benchmark's step: order(), the network-wide build, the forward pass): the
    cached row orders of freed maps and transposed inverses are dropped with
    them, so device memory and the order cache stay flat across steps."""
    from spira_amd.nn.functional import _native
    coords = scenes.indoor(target=120_000, seed=8)   # row orders apply (>= 100k targets)
    model = SparseResUNet42(in_channels=3).to(dev).half().eval()
    spira_amd.nn.fuse_epilogues(model)
    feats = np.random.default_rng(9).standard_normal((len(coords), 3)).astype(np.float32)
    mem, sizes = [], []
    for step in range(10):
        out = _gpu_forward(model, "UNet", coords, feats, dev)
        del out
        torch.cuda.synchronize()
        mem.append(torch.cuda.memory_allocated())
        sizes.append(int(_native._C.row_order_cache_size()))
    print(f"allocated per step (MB): {[round(m / 2**20, 1) for m in mem]}; cached orders: {sizes}", flush=True)
    assert max(mem[3:]) <= mem[2] + (4 << 20), "device memory grows across steps"
    assert max(sizes[3:]) <= sizes[2] + 2, "row-order cache grows across steps"
