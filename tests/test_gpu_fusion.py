"""Fused epilogues (batch norm scale/shift, residual add, ReLU folded into a
conv's output write) on the GPU: every dataflow against the float64 oracle
followed by the same element-wise ops, and whole networks with and without
`fuse_epilogues`.  Tolerance as for the plain layers: max |error| <=
1e-2 * RMS(reference) in fp16, 1e-5 * RMS in fp32.  The network comparison
runs fp32 against fp32, where the fused and unfused paths differ only in
the rounding order of the batch norm (x * scale + shift against
(x - mean) * invstd * weight + bias), which 42 layers amplify: 1e-4 * RMS."""
import copy

import numpy as np
import pytest
import torch

import spira_amd
from oracle import oracle as orc
from spira_amd import scenes
from spira_amd.networks import SparseResUNet42
from spira_amd.nn import functional as F

from helpers import np_, rel_err

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 1e-2, torch.float32: 1e-5}


@pytest.fixture(scope="module")
def keys():
    c = 1 + scenes.spheres_planes(n=4000, grid=64, seed=5)
    k, _ = orc.flatten_sort(c, True)
    return k


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _case(S, T, cin, cout, dtype, dev, seed=3):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(S, cin, generator=g).to(dtype)
    W = (torch.randn(27, cin, cout, generator=g) / np.sqrt(27 * cin)).to(dtype)
    scale = torch.rand(cout, generator=g) + 0.5
    shift = torch.randn(cout, generator=g)
    res = torch.randn(T, cout, generator=g).to(dtype)
    return X, W, scale, shift, res


def _ref(conv, scale, shift, res, relu):
    v = conv * scale.double().numpy() + shift.double().numpy() + res.double().numpy()
    return np.maximum(v, 0) if relu else v


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("dataflow", [0, 1, 2, 3, 4])
@pytest.mark.parametrize("relu", [True, False])
def test_epilogue_every_dataflow(dev, keys, dtype, dataflow, relu):
    S = T = len(keys)
    cin, cout = 32, 64
    X, W, scale, shift, res = _case(S, T, cin, cout, dtype, dev)
    Xn, Wn = X.double().numpy(), W.double().numpy()
    mn = orc.build_kmap(keys, keys, (3, 3, 3), (1, 1, 1), dataflow)
    # each dataflow's own offset order (OS z-major, WS o-major, hybrid L1)
    if dataflow == 0:
        ref_conv = orc.conv_os(mn[2], T, Xn, Wn)
    elif dataflow == 1:
        ref_conv = orc.conv_ws_merged(S, T, Xn, Wn, mn[5], mn[3])
    elif dataflow == 2:
        ref_conv = orc.conv_ws_gs(S, T, Xn, Wn, mn[3], mn[4])
    else:
        dense = orc.conv_os(np.arange(T, dtype=np.int32).reshape(T, 1), T, Xn, Wn[:1])
        ref_conv = (orc.conv_ws_merged(S, T, Xn, Wn, mn[5], mn[3], woffset=1, hybrid=True, Y=dense)
                    if dataflow == 3 else orc.conv_ws_gs(S, T, Xn, Wn, mn[3], mn[4], woffset=1, Y=dense))
    ref = _ref(ref_conv, scale, shift, res, relu)
    epi = (scale.to(dev), shift.to(dev), res.to(dev), relu)
    Xd, Wd = X.to(dev), W.to(dev)
    m = [_t(a, dev) if isinstance(a, np.ndarray) else a for a in mn]
    if dataflow == 0:
        y = F.sparse_convolution_forward_os(S, T, m[2], Xd, Wd, epilogue=epi)
    elif dataflow == 1:
        y = F.sparse_convolution_forward_ws_merged(S, T, Xd, Wd, m[5], m[6], m[3], m[7], m[8], epilogue=epi)
    elif dataflow == 2:
        y = F.sparse_convolution_forward_ws(S, T, Xd, Wd, m[3], m[4], m[5], 16, 16, None, 0.5, epilogue=epi)
    elif dataflow == 3:
        y = F.sparse_convolution_forward_hs_merged(S, T, Xd, Wd, m[5], m[6], m[3], None, m[7], m[8],
                                                   epilogue=epi)
    else:
        y = F.sparse_convolution_forward_hs(S, T, Xd, Wd, m[3], m[4], m[5], None, 16, 16, None, 0.5,
                                            epilogue=epi)
    assert y.dtype == dtype
    assert rel_err(np_(y.float()), ref) <= TOL[dtype]


def _net(dev, dtype, dataflow, seed=0):
    torch.manual_seed(seed)
    model = SparseResUNet42(in_channels=3).to(dev).to(dtype).eval()
    g = torch.Generator().manual_seed(seed + 1)
    for m in model.modules():
        if isinstance(m, spira_amd.nn.BatchNorm):
            n = m.num_features
            m.running_mean.copy_((0.1 * torch.randn(n, generator=g)).to(m.running_mean))
            m.running_var.copy_((0.5 + torch.rand(n, generator=g)).to(m.running_var))
            m.weight.data.copy_((0.5 + torch.rand(n, generator=g)).to(m.weight))
            m.bias.data.copy_((0.1 * torch.randn(n, generator=g)).to(m.bias))
        if isinstance(m, spira_amd.nn.SparseConv):
            m._tunable_config["map_dataflow"] = dataflow
    return model


def _run(model, coords, feats):
    cache = spira_amd.nn.KernelMapCache()
    spira_amd.set_kernel_map_cache(model, cache)
    x = spira_amd.SparseTensor(coordinates=coords, features=feats, double=True)
    x.order()
    with torch.no_grad():
        return [o.features.float() for o in model(x)]


@pytest.mark.parametrize("dataflow", [0, 1, 2])
def test_fused_network_matches_unfused(dev, dataflow):
    coords = torch.from_numpy(1 + scenes.indoor(target=30000, seed=2)).to(dev)
    feats = torch.randn(coords.shape[0], 3, generator=torch.Generator().manual_seed(4)).to(dev)
    plain = _net(dev, torch.float32, dataflow)
    fused = spira_amd.nn.fuse_epilogues(copy.deepcopy(plain))
    ya, yb = _run(plain, coords, feats), _run(fused, coords, feats)
    assert len(ya) == len(yb)
    for a, b in zip(ya, yb):
        assert a.shape == b.shape
        assert rel_err(np_(b), np_(a).astype(np.float64)) <= 1e-4


def test_fused_path_off_with_autograd_or_training(dev):
    coords = torch.from_numpy(1 + scenes.indoor(target=20000, seed=3)).to(dev)
    feats = torch.randn(coords.shape[0], 3, generator=torch.Generator().manual_seed(5)).to(dev)
    model = spira_amd.nn.fuse_epilogues(_net(dev, torch.float32, 0))
    conv = model.stem[0]
    assert conv._epi_bn is model.stem[1] and conv._epi_relu
    with torch.no_grad():
        assert conv._fused_active()
    model.train()
    with torch.no_grad():
        assert not conv._fused_active()
    model.eval()
    with torch.enable_grad():
        assert not conv._fused_active()


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("cin,cout", [(128, 96), (3, 32), (24, 40), (256, 256)])
def test_dense_forward(dev, dtype, cin, cout):
    """1x1x1 layers on the identity-map kernel: sources @ W[0] with the epilogue."""
    T = 3000
    X, W, scale, shift, res = _case(T, T, cin, cout, dtype, dev, seed=7)
    W = W[:1]
    ident = np.arange(T, dtype=np.int32).reshape(T, 1)
    ref_conv = orc.conv_os(ident, T, X.double().numpy(), W.double().numpy())
    y = F.dense_forward(X.to(dev), W.to(dev))
    assert rel_err(np_(y.float()), ref_conv) <= TOL[dtype]
    y = F.dense_forward(X.to(dev), W.to(dev), epilogue=(scale.to(dev), shift.to(dev), res.to(dev), True))
    assert rel_err(np_(y.float()), _ref(ref_conv, scale, shift, res, True)) <= TOL[dtype]


@pytest.mark.parametrize("c1,c2", [(96, 32), (32, 32), (256, 128), (48, 24), (16, 16), (40, 24), (64, 3)])
def test_concat_input_without_copy(dev, keys, c1, c2):
    """A layer whose input is the channel concatenation [A | B] (a decoder's
    skip connection) gathers from the two parts when the split falls on a
    32-channel block, and materialises the concatenation otherwise; both
    match the oracle on the concatenated features, with the epilogue."""
    S = T = len(keys)
    g = torch.Generator().manual_seed(c1 + c2)
    A = torch.randn(S, c1, generator=g).half()
    B = torch.randn(S, c2, generator=g).half()
    W = (torch.randn(27, c1 + c2, 64, generator=g) / np.sqrt(27 * (c1 + c2))).half()
    scale = torch.rand(64, generator=g) + 0.5
    shift = torch.randn(64, generator=g)
    res = torch.randn(T, 64, generator=g).half()
    Xn = torch.cat([A, B], 1).double().numpy()
    m = orc.build_kmap(keys, keys, (3, 3, 3), (1, 1, 1), 0)[2]
    ref_conv = orc.conv_os(m, T, Xn, W.double().numpy())
    epi = (scale.to(dev), shift.to(dev), res.to(dev), True)
    y = F.sparse_convolution_forward_os(S, T, _t(m, dev), A.to(dev), W.to(dev), epilogue=epi, sources2=B.to(dev))
    assert rel_err(np_(y.float()), _ref(ref_conv, scale, shift, res, True)) <= TOL[torch.float16]
    # the 1x1x1 path
    ident = np.arange(T, dtype=np.int32).reshape(T, 1)
    ref_dense = orc.conv_os(ident, T, Xn, W[:1].double().numpy())
    yd = F.dense_forward(A.to(dev), W[:1].to(dev), sources2=B.to(dev))
    assert rel_err(np_(yd.float()), ref_dense) <= TOL[torch.float16]


def test_lazy_cat_materialises_on_access(dev):
    a = spira_amd.SparseTensor(coordinates=torch.zeros(10, dtype=torch.int64, device=dev),
                               features=torch.randn(10, 32, device=dev).half())
    b = spira_amd.SparseTensor(coordinates=a.coordinates, features=torch.randn(10, 16, device=dev).half())
    c = spira_amd.cat([a, b])
    assert c._parts is not None
    assert torch.equal(c.features, torch.cat([a.features, b.features], 1))
    assert c._parts is None
    # splits off a 32-channel block and fp32 parts are concatenated right away
    e = spira_amd.SparseTensor(coordinates=a.coordinates, features=torch.randn(10, 48, device=dev).half())
    d = spira_amd.cat([e, b])
    assert d._parts is None and d.features.shape == (10, 64)
    f = spira_amd.SparseTensor(coordinates=a.coordinates, features=torch.randn(10, 32, device=dev))
    assert spira_amd.cat([f, f])._parts is None
