"""The dataflow selector (reference: source/spira/utils/helpers.py:49-618):
its group rule, the force_os split, the timing accumulator and the on-disk
cache format (a torch.save dict of name_to_group / best_configs /
layer_configs that loads with the weights-only loader).  Which candidate
wins is timing-driven and not pinned; the GPU test checks the group rule and
the cache on a real tuning run."""
import os

import numpy as np
import pytest
import torch

import spira_amd
from spira_amd.networks import SparseResUNet42
from spira_amd.nn import SparseConv
from spira_amd.utils.helpers import (DataflowConfig, StableTimeAccumulator, apply_tuned_configs,
                                     load_tuning_results, save_tuning_results, set_config_for_group)


def _convs(model):
    return [(n, m) for n, m in model.named_modules() if isinstance(m, SparseConv)]


def test_stable_time_accumulator_drops_outliers():
    acc = StableTimeAccumulator()
    for t in (1.0, 1.2, 100.0, 0.8, -1.0):
        acc.add_measurement(t)
    assert acc.get_trial_count() == 3
    assert acc.get_time() == pytest.approx(1.0)


def test_force_os_applies_to_the_first_half_of_a_group():
    model = SparseResUNet42(in_channels=3)
    names = [n for n, m in _convs(model) if m.kernel_size == (3, 3, 3)][:5]
    set_config_for_group(model, names, DataflowConfig(2, True))
    mods = dict(model.named_modules())
    assert [mods[n]._tunable_config["force_os"] for n in names] == [True, True, False, False, False]
    assert all(mods[n]._tunable_config["map_dataflow"] == 2 for n in names)


def test_cache_file_round_trip(tmp_path):
    model = SparseResUNet42(in_channels=3)
    name_to_group = {}
    for n, m in _convs(model):
        name_to_group[n] = ((1, 1, 1), m.kernel_size, m.stride)
    groups = sorted(set(name_to_group.values()))
    best = {g: DataflowConfig(i % 3, i % 2 == 1) for i, g in enumerate(groups)}
    for i, (n, m) in enumerate(_convs(model)):
        m._tunable_config.update(threshold=0.25 * (i % 4), gather_tile_size=8, scatter_tile_size=16,
                                 os_tuning=(32 * (1 + i % 4), 64, i % 3, 1, i % 2, i % 2))
    path = os.path.join(tmp_path, "cfg", "tag.pt")
    requests = {((2, 2, 2), (2, 2, 2), (3, 3, 3)): 1}
    save_tuning_results(name_to_group, best, path, model, requests)
    # the format: plain containers only, readable without unpickling code; the
    # reference's three keys plus this build's per-map row-order requests
    raw = torch.load(path, weights_only=True)
    assert set(raw) == {"name_to_group", "best_configs", "layer_configs", "row_order_requests"}
    assert raw["row_order_requests"] == requests
    assert raw["best_configs"][groups[1]] == {"map_dataflow": 1, "force_os": True}
    n2g, best2, layer_cfgs = load_tuning_results(path)
    assert n2g == name_to_group
    assert {g: (c.map_dataflow, c.force_os) for g, c in best2.items()} == \
        {g: (c.map_dataflow, c.force_os) for g, c in best.items()}
    fresh = SparseResUNet42(in_channels=3)
    apply_tuned_configs(fresh, n2g, best2, layer_cfgs)
    for (n, m), (_, m0) in zip(_convs(fresh), _convs(model)):
        assert m._tunable_config["threshold"] == m0._tunable_config["threshold"]
        assert m._tunable_config["gather_tile_size"] == 8
        assert m._tunable_config["os_tuning"] == m0._tunable_config["os_tuning"]
        assert m._tunable_config["map_dataflow"] == best[name_to_group[n]].map_dataflow
    assert load_tuning_results(path, with_row_orders=True)[3] == requests


def test_os_tuning_changes_the_launch():
    """Every launch field of a layer's tuning reaches the kernel's plan (read
    back through the C ABI, host only), and 0 / None keeps the default."""
    from spira_amd.nn.functional import _native
    C = _native._C
    default = C.conv_os_plan(17044, 27, 256, 0, 256, True)
    assert default == C.conv_os_plan(17044, 27, 256, 0, 256, True, (0, 0, 0, 0, 0, -1))
    assert C.conv_os_plan(17044, 27, 256, 0, 256, True, (96, 0, 0, 0, 0, -1))[0] == 96
    assert C.conv_os_plan(17044, 27, 256, 0, 256, True, (96, 0, 0, 0, 0, -1))[5] == 3  # 256 / 96 column tiles
    assert C.conv_os_plan(17044, 27, 256, 0, 256, True, (0, 32, 0, 0, 0, -1))[1] == 32
    assert C.conv_os_plan(17044, 27, 256, 0, 256, True, (0, 128, 0, 0, 0, -1))[1] == 128
    assert C.conv_os_plan(17044, 27, 256, 0, 256, True, (0, 0, 3, 0, 0, -1))[2] == 3
    # offset packing: 16-channel inputs of 125-offset kernels pack 4 by default
    assert C.conv_os_plan(300000, 125, 16, 0, 16, True)[3] == 4
    assert C.conv_os_plan(300000, 125, 16, 0, 16, True, (0, 0, 0, 1, 0, -1))[3] == 1
    assert C.conv_os_plan(300000, 125, 16, 0, 16, True, (0, 0, 0, 2, 0, -1))[3] == 2
    # (27-offset kernels never pack)
    assert C.conv_os_plan(300000, 27, 16, 0, 16, True, (0, 0, 0, 4, 0, -1))[3] == 1
    assert C.conv_os_plan(17044, 27, 256, 0, 256, True, (0, 0, 0, 0, 1, -1))[6] == 1
    with pytest.raises(RuntimeError, match=r"\[Spira\].*col_tile"):
        C.conv_os_plan(1000, 27, 32, 0, 32, True, (48, 0, 0, 0, 0, -1))


def test_os_candidates():
    from spira_amd.nn.conv import os_candidates
    cols, steps, splits, packs, orders, walks, balance, bpc = os_candidates(256, 256, 27)
    assert cols == [0, 32, 64, 96, 128] and steps == [0, 32, 64, 128] and packs == [0] and orders == [0, 1, 2, 3, 4]
    assert walks == [0]  # the row walk is for inputs of at most 16 channels
    assert balance == [0, 9, 14]  # a third or a half of the offsets per part
    assert bpc == [0, -1, 1, 2]
    cols, steps, splits, packs, orders, walks, balance, bpc = os_candidates(16, 16, 125)
    assert cols == [0, 32] and steps == [0, 32] and packs == [0, 1, 2, 4] and walks == [0, 1]
    assert balance == [0, 42, 63]
    assert os_candidates(3, 32, 1)[2] == [0] and os_candidates(3, 32, 1)[5] == [0]  # no map: no walk
    assert os_candidates(3, 32, 1)[6] == [0]  # nor a balance


@pytest.mark.gpu
def test_tune_on_gpu_groups_and_cache(dev, tmp_path):
    from spira_amd import scenes
    from oracle import oracle as orc
    c = scenes.spheres_planes(n=6000, grid=64, seed=9)
    torch.manual_seed(0)
    # fp32: the same network / dataflow combinations as the fused-network tests
    model = SparseResUNet42(in_channels=3).to(dev).eval()
    cache = spira_amd.nn.KernelMapCache()
    spira_amd.set_kernel_map_cache(model, cache)
    coords = torch.from_numpy(c).to(dev)
    feats = torch.randn(coords.shape[0], 3, device=dev)

    def sample():
        x = spira_amd.SparseTensor(coordinates=coords.clone(), features=feats.clone(), double=True)
        return x.order()

    loader = [sample() for _ in range(5)]
    spira_amd.tune(model, loader, cache, map_dataflow_options=[0, 1, 2], test_force_os=False, n_samples=4,
                   save_dir=str(tmp_path), tune_tag="t", allow_gs_tuning=False)
    path = os.path.join(tmp_path, "t.pt")
    assert os.path.exists(path)
    n2g, best, _ = load_tuning_results(path)
    # every convolution (bar 1x1x1 ones) is in a group; groups with a stride
    # only try dataflows 0-2; a group's layers share their dataflow
    mods = dict(model.named_modules())
    for name, gid in n2g.items():
        if gid in best:
            assert mods[name]._tunable_config["map_dataflow"] == best[gid].map_dataflow
            if any(s > 1 for s in gid[2]):
                assert best[gid].map_dataflow in (0, 1, 2)
    # (the dataflows read the weight rows in their own offset orders, as in the
    # reference, so the tuned network is compared with itself: it runs and is
    # deterministic)
    outs = []
    for _ in range(2):
        with torch.no_grad():
            cache.reset()
            outs.append(model(sample())[-1]._features.float())
    assert torch.isfinite(outs[0]).all() and torch.allclose(outs[0], outs[1], rtol=1e-5, atol=1e-6)
    # a second call loads the cache instead of tuning again
    spira_amd.tune(model, loader, cache, map_dataflow_options=[0], save_dir=str(tmp_path), tune_tag="t",
                   allow_gs_tuning=False)
    n2g2, best2, _ = load_tuning_results(path)
    assert {g: c.map_dataflow for g, c in best2.items()} == {g: c.map_dataflow for g, c in best.items()}


@pytest.mark.gpu
def test_os_tuning_keeps_results(dev, tmp_path):
    """The selector's output-stationary launch choices and row orders change
    the schedule only: a tuned fp16 network gives the untuned network's
    outputs (fp16 storage; fp32 sums in another order, so within the layer
    tolerance 1e-2 x RMS), and every layer that runs the kernel got a choice."""
    from spira_amd import scenes
    from spira_amd.networks import kmap_schedule
    c = scenes.indoor(target=30_000, seed=4)
    torch.manual_seed(1)
    model = SparseResUNet42(in_channels=3)
    g = torch.Generator().manual_seed(2)
    for m in model.modules():
        if isinstance(m, spira_amd.nn.BatchNorm):  # O(1) activations through all levels
            n = m.running_mean.numel()
            m.running_mean.copy_(0.1 * torch.randn(n, generator=g))
            m.running_var.copy_(0.5 + torch.rand(n, generator=g))
            m.weight.data.copy_(0.5 + torch.rand(n, generator=g))
    model = model.to(dev).half().eval()
    spira_amd.nn.fuse_epilogues(model)
    for m in model.modules():
        if isinstance(m, spira_amd.nn.SparseConv):
            m._tunable_config["map_dataflow"] = 0
    cache = spira_amd.nn.KernelMapCache()
    spira_amd.set_kernel_map_cache(model, cache)
    coords = torch.from_numpy(c).to(dev)
    feats = torch.randn(coords.shape[0], 3, device=dev).half()

    def sample():
        x = spira_amd.SparseTensor(coordinates=coords.clone(), features=feats.clone(), double=True)
        return x.order()

    def run():
        cache.reset()
        x = sample()
        ts, ks, ss = kmap_schedule("UNet")
        cache.add_all_kernel_maps(x._coordinates, ks, ss, ts, (1, 1, 1), [0] * len(ks))
        with torch.no_grad():
            return [o._features.float() for o in model(x)]

    before = run()
    spira_amd.tune(model, [sample() for _ in range(3)], cache, map_dataflow_options=[0], test_force_os=False,
                   n_samples=2, save_dir=str(tmp_path), tune_tag="os", allow_gs_tuning=False)
    tuned = [m for m in model.modules() if isinstance(m, spira_amd.nn.SparseConv)
             and m._tunable_config["os_tuning"] is not None]
    assert len(tuned) >= 20 and all(len(m._tunable_config["os_tuning"]) == 9 for m in tuned)
    after = run()
    for a, b in zip(before, after):
        rms = float(a.pow(2).mean().sqrt()) or 1.0
        assert float((a - b).abs().max()) / rms <= 1e-2
