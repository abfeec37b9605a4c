"""Parity at the workloads of the benchmark configurations, full size.

* config 1 -- one fp32 layer, 20k voxels on spheres and planes in a 128^3
  grid, k = 3, C = 32: map bit-exact, features within 1e-5 * RMS on the
  output-stationary, fused weight-stationary and gather-GEMM-scatter
  dataflows;
* config 3 -- the ~100k-voxel LiDAR scene, fp16, k = 3, C = 16 ... 256, every
  dataflow (0 output-stationary, 1 fused weight-stationary, 2
  gather-GEMM-scatter, 3-8 hybrids) against one float64 oracle result per
  width, within 1e-2 * RMS;
* config 4 -- SparseResUNet42 end to end on the 200k-voxel indoor scene with
  the network-wide map build, on dataflow 0 and on the weight-stationary
  dataflows 1 and 2 (the streamed build of pair lists / masks);
* config 5 -- SparseResNetLarge (k = 5) end to end on the ~300k-voxel
  LiDAR-plus-blobs scene.

The reference's end-to-end order is order() -> add_all_kernel_maps -> model
(scripts/end_to_end_experiment.py:194-207).  Network tolerance: the north
star's fp16 bound, max |error| <= 1e-2 * RMS at every output level;
coordinates bit-exact."""
import numpy as np
import pytest
import torch

import spira_amd
from oracle import oracle as orc
from oracle.network import network_forward
from spira_amd import scenes
from spira_amd.networks import SparseResNetLarge, SparseResUNet42, kmap_schedule
from spira_amd.nn import functional as F

from helpers import assert_tuple_equal, np_, rel_err

pytestmark = pytest.mark.gpu

NET_TOL = 1e-2


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _zmajor_of_canonical(kx, ky, kz):
    """zm[j] = canonical offset index of output-stationary column j
    (column iz*O + o  <->  canonical o*kz + iz, O = kx*ky)."""
    O = kx * ky
    return np.array([(j % O) * kz + j // O for j in range(O * kz)], dtype=np.int64)


# ---------------------------------------------------------------- config 1
def test_config1_fp32_layer(dev):
    coords = scenes.spheres_planes(n=20_000, grid=128)
    assert coords.min() >= 0 and coords[:, :2].max() < 4096 and coords[:, 2].max() < 256
    keys, _ = orc.flatten_sort(coords, False)  # 32-bit keys (x12|y12|z8)
    kd = _t(keys, dev)
    S = T = len(keys)
    rng = np.random.default_rng(2026)
    X = rng.standard_normal((S, 32)).astype(np.float32)
    W = (rng.standard_normal((27, 32, 32)) / np.sqrt(27 * 32)).astype(np.float32)
    Xd, Wd = _t(X, dev), _t(W, dev)
    canon = np.ascontiguousarray(orc.search(keys, keys, (3, 3, 3), (1, 1, 1), orc.WS).T)
    ref = orc.conv_os(canon, T, X.astype(np.float64), W.astype(np.float64))
    zm = _zmajor_of_canonical(3, 3, 3)
    for d in (0, 1, 2):
        got = F.build_kmap(kd, kd, 3, 1, d)
        assert_tuple_equal(got, orc.build_kmap(keys, keys, (3, 3, 3), (1, 1, 1), d), f"config 1 dataflow {d}")
        if d == 0:
            y = F.sparse_convolution_forward_os(S, T, got[2], Xd, _t(W[zm], dev))
        elif d == 1:
            y = F.sparse_convolution_forward_ws_merged(S, T, Xd, Wd, got[5], got[6], got[3], got[7], got[8])
        else:
            y = F.sparse_convolution_forward_ws(S, T, Xd, Wd, got[3], got[4], got[5], 16, 16, None, -1)
        assert y.dtype == torch.float32
        err = rel_err(np_(y), ref)
        assert err <= 1e-5, f"config 1 dataflow {d}: error {err:.3g} x RMS"


# ---------------------------------------------------------------- config 3
@pytest.fixture(scope="module")
def lidar():
    keys, _ = orc.flatten_sort(scenes.lidar(), True)
    canon = np.ascontiguousarray(orc.search(keys, keys, (3, 3, 3), (1, 1, 1), orc.WS).T)
    return keys, canon, {}


def _config3_case(lidar, C):
    keys, canon, cache = lidar
    if C not in cache:
        g = torch.Generator().manual_seed(300 + C)
        X = torch.randn(len(keys), C, generator=g).half()
        W = (torch.randn(27, C, C, generator=g) / np.sqrt(27 * C)).half()
        ref = orc.conv_os(canon, len(keys), X.double().numpy(), W.double().numpy())
        cache.clear()  # one width at a time (the oracle result is T x C float64)
        cache[C] = (X, W, ref)
    return cache[C]


@pytest.mark.parametrize("C", [16, 32, 64, 128, 256])
@pytest.mark.parametrize("dataflow", [0, 1, 2])
def test_config3_layer(dev, lidar, C, dataflow):
    keys = lidar[0]
    X, W, ref = _config3_case(lidar, C)
    kd = _t(keys, dev)
    S = T = len(keys)
    m = F.build_kmap(kd, kd, 3, 1, dataflow)
    Xd, Wd = X.to(dev), W.to(dev)
    if dataflow == 0:
        y = F.sparse_convolution_forward_os(S, T, m[2], Xd, W[_zmajor_of_canonical(3, 3, 3)].to(dev))
    elif dataflow == 1:
        y = F.sparse_convolution_forward_ws_merged(S, T, Xd, Wd, m[5], m[6], m[3], m[7], m[8])
    else:
        y = F.sparse_convolution_forward_ws(S, T, Xd, Wd, m[3], m[4], m[5], 16, 16, None, -1)
    err = rel_err(np_(y.float()), ref)
    assert err <= 1e-2, f"config 3 C={C} dataflow {dataflow}: error {err:.3g} x RMS"


@pytest.mark.parametrize("dataflow", [3, 4, 5, 6, 7, 8])
def test_config3_hybrid(dev, lidar, dataflow):
    keys = lidar[0]
    X, W, ref = _config3_case(lidar, 64)
    kd = _t(keys, dev)
    S = T = len(keys)
    m = F.build_kmap(kd, kd, 3, 1, dataflow)
    perm, _ = orc.indexes_l1((3, 3, 3), dataflow)
    # hybrid weight rows: row perm[k] holds canonical offset k
    Wh = W[torch.from_numpy(np.argsort(perm))].to(dev)
    Xd = X.to(dev)
    if dataflow % 2 == 1:
        dense = None if dataflow == 3 else m[2]
        y = F.sparse_convolution_forward_hs_merged(S, T, Xd, Wh, m[5], m[6], m[3], dense, m[7], m[8])
    else:
        dense = None if dataflow == 4 else m[2]
        y = F.sparse_convolution_forward_hs(S, T, Xd, Wh, m[3], m[4], m[5], dense, 16, 16)
    err = rel_err(np_(y.float()), ref)
    assert err <= 1e-2, f"config 3 hybrid {dataflow}: error {err:.3g} x RMS"


# ------------------------------------------------------------ configs 4 / 5
def _randomise_norms(model, seed):
    g = torch.Generator().manual_seed(seed)
    for m in model.modules():
        if isinstance(m, spira_amd.nn.BatchNorm):
            n = m.running_mean.numel()
            m.running_mean.copy_(0.1 * torch.randn(n, generator=g))
            m.running_var.copy_(0.5 + torch.rand(n, generator=g))
            m.weight.data.copy_(0.5 + torch.rand(n, generator=g))
            m.bias.data.copy_(0.1 * torch.randn(n, generator=g))


def _network_case(name, dataflow, dev):
    if name == "UNet":
        coords, model, cin = scenes.indoor(), SparseResUNet42(in_channels=3), 3
    else:
        coords, model, cin = scenes.lidar_blobs(), SparseResNetLarge(in_channels=4), 4
    torch.manual_seed(41)
    _randomise_norms(model, 42)
    model = model.eval().half().float()
    feats = np.random.default_rng(43).standard_normal((len(coords), cin)).astype(np.float32)
    print(f"[{name} dataflow {dataflow}] {len(coords)} voxels: oracle", flush=True)
    ref = network_forward(model, coords, feats, dataflow)
    print(f"[{name} dataflow {dataflow}] GPU", flush=True)
    gpu_model = model.to(dev).half().eval()
    spira_amd.nn.fuse_epilogues(gpu_model)
    for m in gpu_model.modules():
        if isinstance(m, spira_amd.nn.SparseConv):
            m._tunable_config["map_dataflow"] = dataflow
    cache = spira_amd.nn.KernelMapCache()
    spira_amd.set_kernel_map_cache(gpu_model, cache)
    ts, ks, ss = kmap_schedule(name)
    x = spira_amd.SparseTensor(coordinates=torch.from_numpy(coords).to(dev),
                               features=torch.from_numpy(feats).to(dev).half(), double=True)
    x.order()
    cache.add_all_kernel_maps(x._coordinates, ks, ss, ts, (1, 1, 1), [dataflow] * len(ks))
    with torch.no_grad():
        out = gpu_model(x)
    torch.cuda.synchronize()
    rk, _ = orc.flatten_sort(coords, True)
    assert len(out) == len(ref)
    for i, (o, (rf, rs)) in enumerate(zip(out, ref)):
        assert tuple(o.stride) == tuple(rs), f"output {i}: stride {o.stride} != {rs}"
        want = rk if tuple(rs) == (1, 1, 1) else orc.downsample(rk, tuple(rs))
        assert np.array_equal(np_(o.coordinates), want), f"output {i}: coordinates differ"
        assert o.features.shape == rf.shape, f"output {i}: shape {tuple(o.features.shape)} != {rf.shape}"
        err = rel_err(np_(o.features.float()), rf)
        print(f"{name} output {i} stride {tuple(rs)}: max |error| = {err:.3g} x RMS", flush=True)
        assert err <= NET_TOL, f"{name} dataflow {dataflow} output {i} (stride {rs}): error {err:.3g} x RMS"


def test_config4_unet_full(dev):
    _network_case("UNet", 0, dev)


def test_config5_resnet_large_full(dev):
    _network_case("ResNetLarge", 0, dev)


@pytest.mark.parametrize("dataflow", [2, 1])
def test_config4_unet_full_weight_stationary(dev, dataflow):
    _network_case("UNet", dataflow, dev)
