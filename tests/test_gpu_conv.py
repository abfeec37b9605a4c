"""Feature parity on the GPU for every dataflow: outputs of the `_C` feature
entry points against the float64 oracle on the same maps, inputs and weights.
Tolerance: max |error| <= 1e-2 * RMS(reference)
for fp16 storage, <= 1e-5 * RMS(reference) for fp32."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from spira_amd import scenes
from spira_amd.nn import functional as F

from helpers import np_, rel_err

pytestmark = pytest.mark.gpu

TOL = {torch.float16: 1e-2, torch.float32: 1e-5}


@pytest.fixture(scope="module")
def keys():
    # shifted off the origin: there the reference's lower-bound + z-scan drops
    # wrapped entries, and the dataflow-identity checks below need none dropped
    c = 1 + scenes.spheres_planes(n=5000, grid=64, seed=11)
    k, _ = orc.flatten_sort(c, True)
    return k


def _data(S, K, cin, cout, dtype, dev, seed=0):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(S, cin, generator=g)
    W = torch.randn(K, cin, cout, generator=g) / np.sqrt(27 * cin)
    Xd, Wd = X.to(dtype), W.to(dtype)
    # the oracle sees exactly the values stored on the GPU
    return Xd.to(dev), Wd.to(dev), Xd.double().numpy(), Wd.double().numpy()


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


CHANNELS = [(16, 16), (32, 32), (64, 64), (128, 128), (32, 96), (3, 32), (24, 40), (256, 256)]


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("cin,cout", CHANNELS)
def test_os_submanifold(dev, keys, dtype, cin, cout):
    m = orc.build_kmap(keys, keys, (3, 3, 3), (1, 1, 1), 0)
    S = T = len(keys)
    X, W, Xn, Wn = _data(S, 27, cin, cout, dtype, dev)
    y = F.sparse_convolution_forward_os(S, T, _t(m[2], dev), X, W)
    ref = orc.conv_os(m[2], T, Xn, Wn)
    assert y.dtype == dtype and tuple(y.shape) == (T, cout)
    assert rel_err(np_(y.float()), ref) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("cin,cout", [(32, 32), (64, 128), (3, 16)])
def test_ws_merged_submanifold(dev, keys, dtype, cin, cout):
    m = orc.build_kmap(keys, keys, (3, 3, 3), (1, 1, 1), 1)
    S = T = len(keys)
    X, W, Xn, Wn = _data(S, 27, cin, cout, dtype, dev, seed=1)
    y = F.sparse_convolution_forward_ws_merged(S, T, X, W, _t(m[5], dev), _t(m[6], dev), _t(m[3], dev), m[7], m[8])
    ref = orc.conv_ws_merged(S, T, Xn, Wn, m[5], m[3])
    assert rel_err(np_(y.float()), ref) <= TOL[dtype]
    # the mirrored half-map sum equals the full output-stationary sum
    os_ref = orc.conv_os(np.ascontiguousarray(m[2].T), T, Xn, Wn)
    assert rel_err(ref, os_ref) < 1e-12


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("threshold", [-1, 0.5, None])
def test_ws_gather_scatter_submanifold(dev, keys, dtype, threshold):
    m = orc.build_kmap(keys, keys, (3, 3, 3), (1, 1, 1), 2)
    S = T = len(keys)
    X, W, Xn, Wn = _data(S, 27, 64, 64, dtype, dev, seed=2)
    y = F.sparse_convolution_forward_ws(S, T, X, W, _t(m[3], dev), _t(m[4], dev), _t(m[5], dev), 16, 16, None,
                                        threshold)
    ref = orc.conv_ws_gs(S, T, Xn, Wn, m[3], m[4])
    assert rel_err(np_(y.float()), ref) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("dataflow", [3, 4, 5, 6, 7, 8])
def test_hybrid(dev, keys, dtype, dataflow):
    m = orc.build_kmap(keys, keys, (3, 3, 3), (1, 1, 1), dataflow)
    S = T = len(keys)
    X, W, Xn, Wn = _data(S, 27, 32, 32, dtype, dev, seed=3)
    perm, _ = orc.indexes_l1((3, 3, 3), dataflow)
    dense = int(perm[0])
    if dataflow in (3, 4):
        ident = np.arange(T, dtype=np.int32).reshape(T, 1)
        ref = orc.conv_os(ident, T, Xn, Wn[:1])
    else:
        ref = orc.conv_os(m[2], T, Xn, Wn[:dense])
    if dataflow % 2 == 1:
        dmap = None if dataflow == 3 else _t(m[2], dev)
        y = F.sparse_convolution_forward_hs_merged(S, T, X, W, _t(m[5], dev), _t(m[6], dev), _t(m[3], dev), dmap,
                                                   m[7], m[8])
        ref = orc.conv_ws_merged(S, T, Xn, Wn, m[5], m[3], woffset=dense, hybrid=True, Y=ref)
    else:
        dmap = None if dataflow == 4 else _t(m[2], dev)
        y = F.sparse_convolution_forward_hs(S, T, X, W, _t(m[3], dev), _t(m[4], dev), _t(m[5], dev), dmap, 16, 16)
        ref = orc.conv_ws_gs(S, T, Xn, Wn, m[3], m[4], woffset=dense, Y=ref)
    assert rel_err(np_(y.float()), ref) <= TOL[dtype]
    # a hybrid layer with L1-ordered weights equals the canonical convolution
    Wc = Wn[perm]
    full = orc.conv_os(np.ascontiguousarray(orc.search(keys, keys, (3, 3, 3), (1, 1, 1), orc.WS).T), T, Xn, Wc)
    assert rel_err(ref, full) < 1e-12


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("dataflow", [0, 1, 2])
def test_downsample_and_transposed(dev, keys, dtype, dataflow):
    """k=2 stride-2 downsampling conv and the transposed (upsampling) conv that
    reuses its map with sources and targets swapped."""
    tk = orc.downsample(keys, (2, 2, 2))
    m = orc.build_kmap(keys, tk, (2, 2, 2), (1, 1, 1), dataflow)
    S, T = len(keys), len(tk)
    X, W, Xn, Wn = _data(S, 8, 32, 64, dtype, dev, seed=4)
    Xt, Wt, Xtn, Wtn = _data(T, 8, 64, 32, dtype, dev, seed=5)
    if dataflow == 0:
        y = F.sparse_convolution_forward_os(S, T, _t(m[2], dev), X, W)
        ref = orc.conv_os(m[2], T, Xn, Wn)
        tmap = orc.convert_transposed_os(m[2], S)
        yt = F.sparse_convolution_forward_os(T, S, _t(tmap, dev), Xt, Wt)
        reft = orc.conv_os(tmap, S, Xtn, Wtn)
    elif dataflow == 1:
        args = (_t(m[5], dev), _t(m[6], dev), _t(m[3], dev), m[7], m[8])
        y = F.sparse_convolution_forward_ws_merged(S, T, X, W, *args)
        ref = orc.conv_ws_merged(S, T, Xn, Wn, m[5], m[3])
        yt = F.sparse_convolution_forward_ws_merged(T, S, Xt, Wt, *args, True)
        reft = orc.conv_ws_merged(T, S, Xtn, Wtn, m[5], m[3], transpose=True)
    else:
        y = F.sparse_convolution_forward_ws(S, T, X, W, _t(m[3], dev), _t(m[4], dev), _t(m[5], dev), 16, 16)
        ref = orc.conv_ws_gs(S, T, Xn, Wn, m[3], m[4])
        yt = F.sparse_convolution_forward_ws(T, S, Xt, Wt, _t(m[4], dev), _t(m[3], dev), _t(m[5], dev), 16, 16)
        reft = orc.conv_ws_gs(T, S, Xtn, Wtn, m[4], m[3])
    assert rel_err(np_(y.float()), ref) <= TOL[dtype]
    assert rel_err(np_(yt.float()), reft) <= TOL[dtype]


def test_os_k5_large_channels(dev):
    c = scenes.lidar(target=20000, seed=5)
    k, _ = orc.flatten_sort(c, True)
    m = orc.build_kmap(k, k, (5, 5, 5), (1, 1, 1), 0)
    X, W, Xn, Wn = _data(len(k), 125, 128, 128, torch.float16, dev, seed=6)
    y = F.sparse_convolution_forward_os(len(k), len(k), _t(m[2], dev), X, W)
    assert rel_err(np_(y.float()), orc.conv_os(m[2], len(k), Xn, Wn)) <= 1e-2


def test_time_probes(dev, keys):
    m = orc.build_kmap(keys, keys, (3, 3, 3), (1, 1, 1), 2)
    W = torch.randn(27, 32, 32, device=dev, dtype=torch.float16)
    sm, tm, nb = _t(m[3], dev), _t(m[4], dev), _t(m[5], dev)
    for fn in (F.cuda_time_gemm,):
        assert fn(W, sm, tm, nb, threshold=0.5) > 0
    assert F.cuda_time_gather(W, sm, tm, nb, 16) > 0
    assert F.cuda_time_scatter(W, sm, tm, nb, 16) > 0


def test_cpu_tensors_raise(keys):
    x = torch.zeros(4, 4)
    with pytest.raises(NotImplementedError):
        F.sparse_convolution_forward_os(4, 4, torch.zeros(128, 27, dtype=torch.int32), x, torch.zeros(27, 4, 4))


def test_errors_are_runtime_errors(dev):
    X = torch.zeros(10, 16, device=dev, dtype=torch.float16)
    W = torch.zeros(27, 8, 16, device=dev, dtype=torch.float16)  # wrong C_in
    m = torch.full((128, 27), -1, device=dev, dtype=torch.int32)
    with pytest.raises(RuntimeError, match=r"\[Spira\]"):
        F.sparse_convolution_forward_os(10, 10, m, X, W)
