"""Output-stationary layers at full size and the row order they run in: a
200k-voxel indoor scene (row-ordered: targets grouped by neighbour pattern,
the 128-row groups with the most neighbour offsets first) at several widths,
with the fused epilogue, and small layers (fewer blocks than CUs: offsets
split over blocks, fp32 atomics + finalize).  Checked against the float64
oracle on every row; tolerance max |error| <= 1e-2 * RMS(reference) for fp16
storage.  The row order is checked for its defining properties."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from spira_amd import scenes
from spira_amd.nn import functional as F

from helpers import np_, rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def indoor():
    k, _ = orc.flatten_sort(scenes.indoor(), True)
    m = orc.build_kmap(k, k, (3, 3, 3), (1, 1, 1), 0)[2]
    return k, m


def _case(S, cin, cout, dev, seed):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(S, cin, generator=g).half()
    W = (torch.randn(27, cin, cout, generator=g) / np.sqrt(27 * cin)).half()
    return X, W


@pytest.mark.parametrize("cin,cout", [(32, 32), (96, 96), (64, 128), (128, 256)])
def test_ordered_layer(dev, indoor, cin, cout):
    k, m = indoor
    S = T = len(k)
    X, W = _case(S, cin, cout, dev, seed=cin + cout)
    md = torch.from_numpy(m).to(dev)
    y = np_(F.sparse_convolution_forward_os(S, T, md, X.to(dev), W.to(dev)).float())
    ref = orc.conv_os(m, T, X.double().numpy(), W.double().numpy())
    assert rel_err(y, ref) <= 1e-2
    # two calls in a row give the same result up to the fp32 summation order
    y2 = np_(F.sparse_convolution_forward_os(S, T, md, X.to(dev), W.to(dev)).float())
    assert rel_err(y2, y) <= 1e-2


def test_ordered_layer_epilogue(dev, indoor):
    k, m = indoor
    S = T = len(k)
    cin = cout = 96
    X, W = _case(S, cin, cout, dev, seed=5)
    g = torch.Generator().manual_seed(6)
    scale = 0.5 + torch.rand(cout, generator=g)
    shift = 0.1 * torch.randn(cout, generator=g)
    res = torch.randn(T, cout, generator=g).half()
    md = torch.from_numpy(m).to(dev)
    y = F.sparse_convolution_forward_os(S, T, md, X.to(dev), W.to(dev),
                                        epilogue=(scale.to(dev), shift.to(dev), res.to(dev), True))
    conv = orc.conv_os(m, T, X.double().numpy(), W.double().numpy())
    ref = np.maximum(conv * scale.double().numpy() + shift.double().numpy() + res.double().numpy(), 0)
    assert rel_err(np_(y.float()), ref) <= 1e-2


@pytest.mark.parametrize("T,cin,cout", [(300, 64, 64), (2000, 32, 96), (5000, 256, 256), (40, 3, 16)])
def test_small_layer(dev, T, cin, cout):
    c = scenes.spheres_planes(n=T, grid=32, seed=T)
    k, _ = orc.flatten_sort(c, True)
    T = S = len(k)
    m = orc.build_kmap(k, k, (3, 3, 3), (1, 1, 1), 0)[2]
    X, W = _case(S, cin, cout, dev, seed=T)
    y = F.sparse_convolution_forward_os(S, T, torch.from_numpy(m).to(dev), X.to(dev), W.to(dev))
    ref = orc.conv_os(m, T, X.double().numpy(), W.double().numpy())
    assert rel_err(np_(y.float()), ref) <= 1e-2


def _check_row_order(m, T, order, masks, omap):
    K = m.shape[1]
    valid = m[:T] >= 0
    # a permutation of the targets, and the map rows in that order
    assert np.array_equal(np.sort(order), np.arange(T))
    assert np.array_equal(omap, m[order])
    # group masks: the valid-column union of every 128 ordered rows
    G = (T + 127) // 128
    v = np.zeros((G * 128, K), bool)
    v[:T] = valid[order]
    union = v.reshape(G, 128, K).any(1)
    bits = np.zeros((G, 128), bool)
    bits[:, :K] = union
    words = np.packbits(bits.reshape(G, 2, 64)[:, :, ::-1], axis=2, bitorder="big").view(">u8")[:, :, 0]
    assert np.array_equal(masks.view(np.uint64).reshape(G, 2), words.astype(np.uint64))
    # full groups by union size, most columns first; the partial group last
    pc = union.sum(1)
    full = G if T % 128 == 0 else G - 1
    assert np.all(np.diff(pc[:full]) <= 0)
    # inside a group the rows run by neighbour count (most first), then column pattern
    cnt = valid[order].sum(1)
    for g in range(G):
        c = cnt[g * 128:(g + 1) * 128]
        assert np.all(np.diff(c) <= 0)
    if K <= 57:
        # each group is one run of 128 rows of the stable ascending sort of
        # the row keys ((K - count) << K | column mask), in that order
        keys = ((K - valid.sum(1)).astype(np.uint64) << np.uint64(K)) | (
            valid.astype(np.uint64) << np.arange(K, dtype=np.uint64)).sum(1, dtype=np.uint64)
        srt = np.argsort(keys, kind="stable")
        runs = {int(srt[i]): srt[i:i + 128] for i in range(0, T, 128)}
        for g in range(G):
            grp = order[g * 128:(g + 1) * 128]
            assert np.array_equal(grp, runs[int(grp[0])])


def test_row_order_k3(dev, indoor):
    from spira_amd.nn.functional._native import _C
    k, m = indoor
    T = len(k)
    order, masks, omap = (np_(t) for t in _C.kmap_row_order(torch.from_numpy(m).to(dev), T))
    _check_row_order(m, T, order, masks, omap)


@pytest.mark.parametrize("T", [1, 130, 2048, 3001])
def test_row_order_small(dev, indoor, T):
    """Sort tiles of 2048 rows: one partial tile, exactly one, and a partial second."""
    from spira_amd.nn.functional._native import _C
    m = np.ascontiguousarray(indoor[1][:T])
    order, masks, omap = (np_(t) for t in _C.kmap_row_order(torch.from_numpy(m).to(dev), T))
    _check_row_order(m, T, order, masks, omap)


def test_row_order_k5(dev):
    from spira_amd.nn.functional._native import _C
    c = scenes.spheres_planes(n=20000, grid=64, seed=3)
    k, _ = orc.flatten_sort(c, True)
    T = len(k) - 77  # a partial last group
    m = orc.build_kmap(k, k, (5, 5, 5), (1, 1, 1), 0)[2]
    order, masks, omap = (np_(t) for t in _C.kmap_row_order(torch.from_numpy(m).to(dev), T))
    _check_row_order(m, T, order, masks, omap)


@pytest.fixture(scope="module")
def scene_k5():
    c = scenes.spheres_planes(n=60000, grid=96, seed=9)
    k, _ = orc.flatten_sort(c, True)
    return k, orc.build_kmap(k, k, (5, 5, 5), (1, 1, 1), 0)[2]


@pytest.mark.parametrize("ks,cin,cout", [(3, 16, 32), (3, 24, 40), (3, 32, 64), (3, 8, 16),
                                         (5, 16, 16), (5, 32, 32), (5, 24, 96), (5, 64, 64), (5, 56, 32)])
def test_offset_packing(dev, indoor, scene_k5, ks, cin, cout):
    """16- and 32-channel (padded) inputs of kernels with more than 27
    offsets run four kernel offsets per step: 125 offsets leave the last step
    with one, and rows without a neighbour at one of a step's offsets must
    read zeros there.  k = 3 on the 200k scene (map tile in LDS, one offset
    per step) for comparison."""
    k, m = indoor if ks == 3 else scene_k5
    S = T = len(k)
    X = _case(S, cin, cout, dev, seed=ks * 100 + cin)[0]
    g = torch.Generator().manual_seed(cin + cout)
    W = (torch.randn(m.shape[1], cin, cout, generator=g) / np.sqrt(m.shape[1] * cin)).half()
    md = torch.from_numpy(m).to(dev)
    y = np_(F.sparse_convolution_forward_os(S, T, md, X.to(dev), W.to(dev)).float())
    ref = orc.conv_os(m, T, X.double().numpy(), W.double().numpy())
    assert rel_err(y, ref) <= 1e-2


_PACK_CHILD = """
import sys
import numpy as np
import torch
sys.path.insert(0, "tests")
from oracle import oracle as orc
from spira_amd import scenes
from spira_amd.nn import functional as F
from helpers import rel_err
c = scenes.spheres_planes(n=60000, grid=96, seed=9)
k, _ = orc.flatten_sort(c, True)
T = len(k)
g = torch.Generator().manual_seed(1)
worst = 0.0
for ks in (3, 5):
    m = orc.build_kmap(k, k, (ks, ks, ks), (1, 1, 1), 0)[2]
    K = m.shape[1]
    for cin, cout in [(16, 32), (32, 32), (24, 64), (64, 64)]:
        X = torch.randn(T, cin, generator=g).half()
        W = (torch.randn(K, cin, cout, generator=g) / np.sqrt(K * cin)).half()
        y = F.sparse_convolution_forward_os(T, T, torch.from_numpy(m).cuda(), X.cuda(), W.cuda())
        ref = orc.conv_os(m, T, X.double().numpy(), W.double().numpy())
        worst = max(worst, rel_err(y.float().cpu().numpy(), ref))
print("WORST", worst)
"""


@pytest.mark.parametrize("pack", ["2", "0"])
def test_offset_packing_variants(dev, pack):
    """Pairs of offsets per step (SPIRA_OS_PACK=2) and no packing (=0), k = 3
    and 5, each in a child process since the library reads SPIRA_OS_PACK
    once."""
    import os
    import subprocess
    import sys
    env = dict(os.environ, SPIRA_OS_PACK=pack)
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, "-c", _PACK_CHILD], env=env, cwd=root, capture_output=True, text=True,
                       timeout=150)
    assert r.returncode == 0, r.stderr[-2000:]
    assert float(r.stdout.split("WORST")[-1]) <= 1e-2


def _check_small_row_order(m, T, order, masks, omap):
    """Maps of <= 8 offsets: the order is exactly the stable sort of the rows
    by (neighbour count descending, column mask ascending), with the map rows
    and the exact 128-row column unions in that order."""
    K = m.shape[1]
    valid = m[:T] >= 0
    key = ((K - valid.sum(1)) << K) | (valid * (1 << np.arange(K))).sum(1)
    assert np.array_equal(order, np.argsort(key, kind="stable"))
    assert np.array_equal(omap, m[order])
    G = (T + 127) // 128
    v = np.zeros((G * 128, K), bool)
    v[:T] = valid[order]
    union = (v.reshape(G, 128, K).any(1) * (1 << np.arange(K))).sum(1)
    assert np.array_equal(masks.view(np.uint64).reshape(G, 2)[:, 0], union.astype(np.uint64))
    assert not masks.view(np.uint64).reshape(G, 2)[:, 1].any()


def test_row_order_k2_maps(dev, indoor):
    """The k = 2 down-sampling map of the config-4 scene and its transpose
    (one valid entry per row: the counting-sort path)."""
    from spira_amd.nn.functional._native import _C
    k = indoor[0]
    k2 = orc.downsample(k, (2, 2, 2))
    m = np.ascontiguousarray(orc.build_kmap(k, k2, (2, 2, 2), (1, 1, 1), 0)[2])
    for mm, T in ((m, len(k2)), (np.ascontiguousarray(orc.convert_transposed_os(m, len(k))), len(k))):
        order, masks, omap = (np_(t) for t in _C.kmap_row_order(torch.from_numpy(mm).to(dev), T))
        _check_small_row_order(mm, T, order, masks, omap)


@pytest.mark.parametrize("T,K", [(1, 8), (1000, 8), (1024, 8), (1025, 4), (5000, 8), (70000, 2)])
def test_row_order_small_maps(dev, T, K):
    """Random maps of <= 8 offsets around the 1024-row tiles of the counting sort."""
    from spira_amd.nn.functional._native import _C
    rng = np.random.default_rng(T + K)
    m = np.where(rng.random((T, K)) < 0.4, rng.integers(0, 1000, (T, K)), -1).astype(np.int32)
    order, masks, omap = (np_(t) for t in _C.kmap_row_order(torch.from_numpy(m).to(dev), T))
    _check_small_row_order(m, T, order, masks, omap)


@pytest.mark.parametrize("transposed", [False, True])
def test_ordered_k2_layer(dev, indoor, transposed):
    """A k = 2 stride-2 layer and its transpose walked in row order (the
    layer's tuning asks for it) against the oracle."""
    k = indoor[0]
    k2 = orc.downsample(k, (2, 2, 2))
    m = orc.build_kmap(k, k2, (2, 2, 2), (1, 1, 1), 0)[2]
    S, T = len(k), len(k2)
    if transposed:
        m, S, T = orc.convert_transposed_os(m, S), T, S
    X, W = _case(S, 96, 96, dev, seed=11)
    W = W[:8].contiguous()
    md = torch.from_numpy(np.ascontiguousarray(m)).to(dev)
    ref = orc.conv_os(m, T, X.double().numpy(), W.double().numpy())
    for rows in (1, 0):
        y = F.sparse_convolution_forward_os(S, T, md, X.to(dev), W.to(dev), tuning=(0, 0, 0, 0, 0, rows))
        assert rel_err(np_(y.float()), ref) <= 1e-2, rows


@pytest.mark.parametrize("ks,cin,cout", [(3, 3, 32), (3, 8, 24), (3, 16, 16), (5, 4, 16), (5, 16, 16), (5, 16, 32),
                                         (5, 11, 40)])
def test_row_walk(dev, indoor, scene_k5, ks, cin, cout):
    """The per-target row walk (tuning row_walk = 1: few input channels on
    the vector ALU) against the oracle, with the fused epilogue, on the
    config-4 k=3 map and a k=5 map; C_in up to 16, any C_out."""
    k, m = indoor if ks == 3 else scene_k5
    S = T = len(k)
    K = ks ** 3
    g = torch.Generator().manual_seed(cin * 100 + cout)
    X = torch.randn(S, cin, generator=g).half()
    W = (torch.randn(K, cin, cout, generator=g) / np.sqrt(K * cin)).half()
    scale = 0.5 + torch.rand(cout, generator=g)
    shift = 0.1 * torch.randn(cout, generator=g)
    res = torch.randn(T, cout, generator=g).half()
    md = torch.from_numpy(m).to(dev)
    conv = orc.conv_os(m, T, X.double().numpy(), W.double().numpy())
    y = F.sparse_convolution_forward_os(S, T, md, X.to(dev), W.to(dev), tuning=(0, 0, 0, 0, 0, -1, 1))
    assert rel_err(np_(y.float()), conv) <= 1e-2
    ye = F.sparse_convolution_forward_os(S, T, md, X.to(dev), W.to(dev), tuning=(0, 0, 0, 0, 0, -1, 1),
                                         epilogue=(scale.to(dev), shift.to(dev), res.to(dev), True))
    ref = np.maximum(conv * scale.double().numpy() + shift.double().numpy() + res.double().numpy(), 0)
    assert rel_err(np_(ye.float()), ref) <= 1e-2


# Launches that issue the gathered rows two steps ahead of the weights (64-
# and 128-channel steps of 96- and 128-column tiles whose grid is too large
# for a third LDS stage: 200k rows): index and row order, block orders, a
# channel concatenation, and an output width that leaves a partial column
# tile.  (tuning: col_tile, step_channels, offset_splits, offset_pack,
# block_order, row_order)
@pytest.mark.parametrize("cin,cout,tuning", [
    (128, 128, (128, 128, 0, 0, 0, 1)),
    (128, 128, (128, 64, 0, 0, 4, 0)),
    (96, 96, (96, 128, 0, 0, 1, 1)),
    (96, 96, (96, 64, 0, 0, 2, 1)),
    (128, 160, (96, 128, 0, 0, 0, 0)),
])
def test_two_step_gathers(dev, indoor, cin, cout, tuning):
    k, m = indoor
    S = T = len(k)
    X, W = _case(S, cin, cout, dev, seed=cin * 7 + cout)
    md = torch.from_numpy(m).to(dev)
    y = np_(F.sparse_convolution_forward_os(S, T, md, X.to(dev), W.to(dev), tuning=tuning).float())
    ref = orc.conv_os(m, T, X.double().numpy(), W.double().numpy())
    assert rel_err(y, ref) <= 1e-2


def test_two_step_gathers_concat(dev, indoor):
    k, m = indoor
    S = T = len(k)
    X, W = _case(S, 192, 128, dev, seed=11)
    md = torch.from_numpy(m).to(dev)
    Xd = X.to(dev)
    y = np_(F.sparse_convolution_forward_os(S, T, md, Xd[:, :128].contiguous(), W.to(dev),
                                            sources2=Xd[:, 128:].contiguous(), tuning=(128, 128, 0, 0, 0, 1)).float())
    ref = orc.conv_os(m, T, X.double().numpy(), W.double().numpy())
    assert rel_err(y, ref) <= 1e-2


# Work balance (tuning balance_offsets, the eighth field): on a row-ordered
# map, a row tile with more valid offsets than the field is split over
# several blocks whose fp32 partial tiles a second pass sums.  Checked
# against the oracle at the benchmark's stride-8 level (the most neighbours
# per row) and at stride 1, with the fused epilogue and a channel
# concatenation; repeated calls give identical outputs (the parts are summed
# in a fixed order), and the workspace comes back zeroed (an offset-split
# call on the same workspace right after still matches the oracle).
@pytest.fixture(scope="module")
def indoor_s8():
    k, _ = orc.flatten_sort(scenes.indoor(), True)
    k8 = orc.downsample(k, (8, 8, 8))
    m = orc.build_kmap(k8, k8, (3, 3, 3), (8, 8, 8), 0)[2]
    return k8, m


@pytest.mark.parametrize("cin,cout,tuning", [
    (256, 256, (128, 128, 0, 0, 0, 1, 0, 9)),
    (256, 256, (96, 128, 0, 0, 0, 1, 0, 5)),
    (128, 128, (0, 64, 0, 0, 2, 1, 0, 9)),
    (64, 96, (0, 0, 0, 0, 0, 1, 0, 3)),
])
def test_balanced_layer(dev, indoor_s8, cin, cout, tuning):
    k, m = indoor_s8
    S = T = len(k)
    X, W = _case(S, cin, cout, dev, seed=cin + 3 * cout)
    md = torch.from_numpy(m).to(dev)
    y = F.sparse_convolution_forward_os(S, T, md, X.to(dev), W.to(dev), tuning=tuning)
    ref = orc.conv_os(m, T, X.double().numpy(), W.double().numpy())
    assert rel_err(np_(y.float()), ref) <= 1e-2
    y2 = F.sparse_convolution_forward_os(S, T, md, X.to(dev), W.to(dev), tuning=tuning)
    assert torch.equal(y, y2)
    # the same layer with its offsets split over blocks (fp32 atomics into
    # the workspace, which must have come back zeroed)
    y3 = F.sparse_convolution_forward_os(S, T, md, X.to(dev), W.to(dev), tuning=(0, 0, 4, 0, 0, 1, 0, -1))
    assert rel_err(np_(y3.float()), ref) <= 1e-2


def test_balanced_layer_epilogue_concat(dev, indoor_s8):
    k, m = indoor_s8
    S = T = len(k)
    cout = 256
    X, W = _case(S, 384, cout, dev, seed=21)
    g = torch.Generator().manual_seed(22)
    scale = 0.5 + torch.rand(cout, generator=g)
    shift = 0.1 * torch.randn(cout, generator=g)
    res = torch.randn(T, cout, generator=g).half()
    md = torch.from_numpy(m).to(dev)
    Xd = X.to(dev)
    y = F.sparse_convolution_forward_os(S, T, md, Xd[:, :256].contiguous(), W.to(dev),
                                        epilogue=(scale.to(dev), shift.to(dev), res.to(dev), True),
                                        sources2=Xd[:, 256:].contiguous(), tuning=(128, 128, 0, 0, 0, 1, 0, 9))
    conv = orc.conv_os(m, T, X.double().numpy(), W.double().numpy())
    ref = np.maximum(conv * scale.double().numpy() + shift.double().numpy() + res.double().numpy(), 0)
    assert rel_err(np_(y.float()), ref) <= 1e-2


def test_balanced_layer_full_size(dev, indoor):
    k, m = indoor
    S = T = len(k)
    X, W = _case(S, 96, 96, dev, seed=31)
    md = torch.from_numpy(m).to(dev)
    y = np_(F.sparse_convolution_forward_os(S, T, md, X.to(dev), W.to(dev), tuning=(0, 0, 0, 0, 0, 1, 0, 3)).float())
    ref = orc.conv_os(m, T, X.double().numpy(), W.double().numpy())
    assert rel_err(y, ref) <= 1e-2
