"""Every `_C` function called exactly as the reference's Python layer calls it:
the same positional arguments and nothing else (reference call sites:
spira/nn/functional/indexing.py:25-105, convolution.py:27-172, memory.py:8-11;
declarations: csrc/spira/torch/cuda_*.cu).  Each result is checked against the
oracle: maps and coordinates bit for bit, features within 1e-2 * RMS (fp16)."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from spira_amd import scenes
from spira_amd.nn.functional import _native

from helpers import assert_tuple_equal, np_, rel_err

pytestmark = pytest.mark.gpu

_C = _native._C
TOL = 1e-2


@pytest.fixture(scope="module")
def scene():
    # shifted off the origin so that no lookup wraps around 2^64
    return 1 + scenes.spheres_planes(n=5000, grid=64, seed=21)


@pytest.fixture(scope="module")
def keys(scene):
    k, _ = orc.flatten_sort(scene, True)
    return k


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _feat(S, K, cin, cout, dev, seed):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(S, cin, generator=g).half()
    W = (torch.randn(K, cin, cout, generator=g) / np.sqrt(27 * cin)).half()
    return X.to(dev), W.to(dev), X.double().numpy(), W.double().numpy()


def test_index_functions_at_reference_arity(dev, scene, keys):
    c = _t(scene, dev)
    for double in (False, True):
        k, perm = _C.cuda_flatten_sort(c, double)                      # indexing.py:25
        rk, rp = orc.flatten_sort(scene, double)
        assert np.array_equal(np_(k), rk) and np.array_equal(np_(perm).astype(np.int64), rp.astype(np.int64))
        assert np.array_equal(np_(_C.cuda_unflatten(k)), orc.unflatten(rk))   # indexing.py:32
    tk = _t(keys, dev)
    assert np.array_equal(np_(_C.cuda_downsample(tk, 2, 2, 2)), orc.downsample(keys, (2, 2, 2)))  # indexing.py:61
    strides = [(2, 2, 2), (4, 4, 4)]
    outs = _C.cuda_streamed_output_generate(tk, strides)               # indexing.py:38
    for o, s in zip(outs, strides):
        assert np.array_equal(np_(o), orc.downsample(keys, s))
    for df in range(9):                                                 # indexing.py:77
        got = _C.cuda_binary_search(tk, tk, (3, 3, 3), (1, 1, 1), df)
        assert_tuple_equal(got, orc.build_kmap(keys, keys, (3, 3, 3), (1, 1, 1), df), f"dataflow {df}")
    got = _C.cuda_binary_search_no_small_z(tk, tk, (3, 3, 3), (1, 1, 1))  # indexing.py:105
    assert_tuple_equal(got, orc.build_kmap_no_small_z(keys, keys, (3, 3, 3), (1, 1, 1)), "no_small_z")
    coarse = orc.downsample(keys, (2, 2, 2))
    vox = [tk, _t(coarse, dev)]
    maps = _C.cuda_binary_search_streamed(vox, [(3, 3, 3), (2, 2, 2)], [(1, 1, 1), (1, 1, 1)], [0, 1])  # indexing.py:56
    assert_tuple_equal(maps[0], orc.build_kmap(keys, keys, (3, 3, 3), (1, 1, 1), 0), "streamed 0")
    assert_tuple_equal(maps[1], orc.build_kmap(keys, coarse, (2, 2, 2), (1, 1, 1), 1, half=False), "streamed 1")
    m = orc.build_kmap(keys, coarse, (2, 2, 2), (1, 1, 1), 0)[2]
    inv = _C.cuda_convert_transposed_os(_t(m, dev), len(keys))         # indexing.py:86
    assert np.array_equal(np_(inv), orc.convert_transposed_os(m, len(keys)))


def test_forward_functions_at_reference_arity(dev, keys):
    S = T = len(keys)
    X, W, Xn, Wn = _feat(S, 27, 32, 32, dev, seed=5)
    # dataflow 0 (convolution.py:172)
    m0 = orc.build_kmap(keys, keys, (3, 3, 3), (1, 1, 1), 0)
    y = _C.cuda_sparse_convolution_forward_os(S, T, _t(m0[2], dev), X, W)
    assert rel_err(np_(y.float()), orc.conv_os(m0[2], T, Xn, Wn)) <= TOL
    # dataflow 1 (convolution.py:101)
    m1 = orc.build_kmap(keys, keys, (3, 3, 3), (1, 1, 1), 1)
    y = _C.cuda_sparse_convolution_forward_ws_merged(S, T, X, W, _t(m1[5], dev), _t(m1[6], dev), _t(m1[3], dev),
                                                     m1[7], m1[8], False)
    assert rel_err(np_(y.float()), orc.conv_ws_merged(S, T, Xn, Wn, m1[5], m1[3])) <= TOL
    # dataflow 2 (convolution.py:78), threshold None / 0 / -1 as the reference passes them
    m2 = orc.build_kmap(keys, keys, (3, 3, 3), (1, 1, 1), 2)
    ref2 = orc.conv_ws_gs(S, T, Xn, Wn, m2[3], m2[4])
    for thr in (None, 0.0, -1.0):
        y = _C.cuda_sparse_convolution_forward_ws(S, T, 16, 16, 4, thr, X, W, _t(m2[3], dev), _t(m2[4], dev),
                                                  _t(m2[5], dev))
        assert rel_err(np_(y.float()), ref2) <= TOL, f"threshold {thr}"


@pytest.mark.parametrize("dataflow", [3, 4, 5, 6, 7, 8])
def test_hybrid_forward_at_reference_arity(dev, keys, dataflow):
    S = T = len(keys)
    X, W, Xn, Wn = _feat(S, 27, 32, 32, dev, seed=6)
    m = orc.build_kmap(keys, keys, (3, 3, 3), (1, 1, 1), dataflow)
    perm, _ = orc.indexes_l1((3, 3, 3), dataflow)
    dense = int(perm[0])
    if dataflow in (3, 4):
        ref = orc.conv_os(np.arange(T, dtype=np.int32).reshape(T, 1), T, Xn, Wn[:1])
        dmap = None
    else:
        ref = orc.conv_os(m[2], T, Xn, Wn[:dense])
        dmap = _t(m[2], dev)
    if dataflow % 2 == 1:   # convolution.py:158
        y = _C.cuda_sparse_convolution_forward_hs_merged(S, T, X, W, _t(m[5], dev), _t(m[6], dev), _t(m[3], dev),
                                                         dmap, m[7], m[8], False)
        ref = orc.conv_ws_merged(S, T, Xn, Wn, m[5], m[3], woffset=dense, hybrid=True, Y=ref)
    else:                   # convolution.py:132
        y = _C.cuda_sparse_convolution_forward_hs(S, T, 16, 16, 4, 0.0, X, W, _t(m[3], dev), _t(m[4], dev),
                                                  _t(m[5], dev), dmap)
        ref = orc.conv_ws_gs(S, T, Xn, Wn, m[3], m[4], woffset=dense, Y=ref)
    assert rel_err(np_(y.float()), ref) <= TOL


def test_timing_and_memory_functions_at_reference_arity(dev, keys):
    m = orc.build_kmap(keys, keys, (3, 3, 3), (1, 1, 1), 2)
    W = torch.randn(27, 32, 32, device=dev).half()
    sm, tm, nb = _t(m[3], dev), _t(m[4], dev), _t(m[5], dev)
    # convolution.py:27-55: (parallel | tile, threshold, is_hybrid, W, masks, masks, sizes)
    assert _C.cuda_time_gemm(4, 0.5, False, W, sm, tm, nb) > 0
    assert _C.cuda_time_gather(16, None, False, W, sm, tm, nb) > 0
    assert _C.cuda_time_scatter(16, -1.0, False, W, sm, tm, nb) > 0
    assert _C.cuda_free_buffers() is None        # memory.py:8
    assert _C.cuda_reset_error() is None         # memory.py:11
