"""Kernel-map parity on the GPU: every element of the `_C` 9-tuples must be
bit-identical to the oracle (oracle/oracle.py, itself pinned by
tests/test_oracle.py).  Runs through spira_amd's `_C` -> libspira_hip.so."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from spira_amd import scenes
from spira_amd.nn import functional as F

from helpers import assert_tuple_equal, np_, rel_err

pytestmark = pytest.mark.gpu


def _keys(coords, bits, dev):
    k, _ = orc.flatten_sort(coords, bits == 64)
    return k, torch.from_numpy(k).to(dev)


@pytest.fixture(scope="module")
def scene_small():
    return scenes.spheres_planes(n=6000, grid=64, seed=7)


@pytest.fixture(scope="module")
def scene_lidar():
    return scenes.lidar()


def test_flatten_sort_and_unflatten(dev, scene_small):
    for double in (False, True):
        c = torch.from_numpy(scene_small).to(dev)
        keys, perm = F.flat_sort(c, double)
        rk, rp = orc.flatten_sort(scene_small, double)
        assert np.array_equal(np_(keys), rk)
        assert np.array_equal(np_(perm), rp.astype(np.int64))
        assert np.array_equal(np_(F.unflatten(keys)), orc.unflatten(rk))


@pytest.mark.parametrize("double", [True, False])
def test_flatten_sort_large(dev, double):
    """A large shuffled input (over 300k rows, a third of them repeated):
    keys and the stable permutation against the oracle (equal keys keep
    their input order)."""
    rng = np.random.default_rng(5)
    c = np.unique(rng.integers(0, 250, size=(420000, 3)), axis=0).astype(np.int32)
    c = rng.permutation(np.concatenate([c, c[::3]]))
    assert c.shape[0] > 250000
    keys, perm = F.flat_sort(torch.from_numpy(c).to(dev), double)
    rk, rp = orc.flatten_sort(c, double)
    assert np.array_equal(np_(keys), rk)
    assert np.array_equal(np_(perm), rp.astype(np.int64))


def test_flatten_sort_duplicates_are_stable(dev):
    rng = np.random.default_rng(3)
    c = rng.integers(0, 6, size=(5000, 3)).astype(np.int32)  # many duplicates
    keys, perm = F.flat_sort(torch.from_numpy(c).to(dev), True)
    rk, rp = orc.flatten_sort(c, True)
    assert np.array_equal(np_(keys), rk)
    assert np.array_equal(np_(perm), rp.astype(np.int64))


@pytest.mark.parametrize("bits", [32, 64])
@pytest.mark.parametrize("stride", [(2, 2, 2), (4, 4, 4), (1, 1, 2), (8, 8, 16)])
def test_downsample(dev, scene_small, bits, stride):
    rk, tk = _keys(scene_small, bits, dev)
    got = F.downsample(tk, stride)
    assert np.array_equal(np_(got), orc.downsample(rk, stride))


def test_streamed_output_generate(dev, scene_small):
    rk, tk = _keys(scene_small, 64, dev)
    strides = [(2, 2, 2), (4, 4, 4), (8, 8, 8), (16, 16, 16)]
    outs = F.streamed_output_generate(tk, strides)
    for o, s in zip(outs, strides):
        assert np.array_equal(np_(o), orc.downsample(rk, s))


def _grid(xs, ys, zs):
    g = np.stack(np.meshgrid(np.asarray(xs), np.asarray(ys), np.asarray(zs), indexing="ij"), -1)
    return g.reshape(-1, 3).astype(np.int32)


# Target-stride lists whose strides nest (powers of two, each a multiple of
# the previous one): the streamed call takes the chained path (each level from
# the previous one, no host read); unsorted keys fall back to the per-stride
# path.  The anisotropic list merges 2 x 4 input rows per output run.
CHAINS = [[(2, 2, 2), (4, 4, 4), (8, 8, 16), (16, 16, 16)], [(1, 1, 2), (2, 2, 2), (4, 8, 8)],
          [(1, 1, 1), (4, 4, 4)]]


def _ds_case(dev, keys_np, bits, strides, chains=()):
    tk = torch.from_numpy(keys_np).to(dev)
    for s in strides:
        assert np.array_equal(np_(F.downsample(tk, s)), orc.downsample(keys_np, s)), s
    for lst in [strides, *chains]:
        outs = F.streamed_output_generate(tk, lst)
        assert len(outs) == len(lst)
        for o, s in zip(outs, lst):
            assert np.array_equal(np_(o), orc.downsample(keys_np, s)), (lst, s)


@pytest.mark.parametrize("bits", [32, 64])
def test_downsample_paths(dev, bits):
    """Each downsample path against the oracle, for single and streamed calls:
    the segmented path with 32-bit sort keys (runs of equal masked x up to 4k
    and up to 16k keys), the general path for unsorted keys and for a run
    longer than 32768 keys (one dense x plane), sorted keys with duplicates,
    and one or two keys."""
    strides = [(2, 2, 2), (4, 4, 4), (1, 1, 2), (8, 8, 16), (1, 1, 1)]
    rng = np.random.default_rng(21)
    scattered = np.unique(rng.integers(0, 200, size=(30000, 3)), axis=0).astype(np.int32)
    scattered[:, 2] %= 200 if bits == 64 else 250
    plane = _grid([3], range(0, 200), range(0, 200 if bits == 64 else 250))  # 40k-50k keys in one x run
    slab = _grid([4, 5], range(0, 85), range(0, 85))  # 14450 keys in one run at x stride 2
    for c in (scattered, np.concatenate([scattered, slab]), np.concatenate([scattered, plane])):
        rk, _ = orc.flatten_sort(c, bits == 64)
        _ds_case(dev, rk, bits, strides, CHAINS)
        _ds_case(dev, rng.permutation(rk), bits, strides, CHAINS)  # unsorted
        _ds_case(dev, np.sort(np.concatenate([rk, rk[::3]])), bits, strides, CHAINS)  # duplicates
    for c in (scattered[:1], scattered[:2]):
        rk, _ = orc.flatten_sort(c, bits == 64)
        _ds_case(dev, rk, bits, strides, CHAINS)


def test_downsample_wide_sort_keys(dev):
    """Negative y makes the varying bits below x wider than 32 (64-bit keys):
    the segmented path with 64-bit sort keys (runs up to 4k and 16k keys)."""
    rng = np.random.default_rng(22)
    pts = np.unique(rng.integers(-300, 300, size=(40000, 3)), axis=0).astype(np.int32)
    pts[:, 2] = np.abs(pts[:, 2])
    slab = _grid([-2, -1], range(-40, 41), range(0, 91))  # 14742 keys in one x run at stride 2
    for c in (pts, np.concatenate([pts, slab])):
        rk, _ = orc.flatten_sort(np.unique(c, axis=0), True)
        _ds_case(dev, rk, 64, [(2, 2, 2), (4, 4, 4), (1, 2, 1), (16, 16, 16)], CHAINS)


def test_downsample_indoor_scene(dev):
    """Config-4 scene: runs of up to ~16.5k keys (the 32k-key block tile)."""
    rk, _ = orc.flatten_sort(scenes.indoor(), True)
    _ds_case(dev, rk, 64, [(2, 2, 2), (4, 4, 4), (8, 8, 8), (16, 16, 16)], CHAINS)


@pytest.mark.parametrize("bits", [32, 64])
@pytest.mark.parametrize("dataflow", list(range(9)))
def test_submanifold_all_dataflows(dev, scene_small, bits, dataflow):
    rk, tk = _keys(scene_small, bits, dev)
    got = F.build_kmap(tk, tk, 3, 1, dataflow)
    ref = orc.build_kmap(rk, rk, (3, 3, 3), (1, 1, 1), dataflow)
    assert_tuple_equal(got, ref, f"bits={bits} dataflow={dataflow}")


@pytest.mark.parametrize("dataflow", [0, 1, 2, 3, 4, 5, 6, 7, 8])
def test_submanifold_k5(dev, scene_small, dataflow):
    rk, tk = _keys(scene_small, 64, dev)
    got = F.build_kmap(tk, tk, 5, 1, dataflow)
    ref = orc.build_kmap(rk, rk, (5, 5, 5), (1, 1, 1), dataflow)
    assert_tuple_equal(got, ref, f"k5 dataflow={dataflow}")


@pytest.mark.parametrize("bits", [32, 64])
@pytest.mark.parametrize("ksize", [(2, 2, 2), (3, 3, 3), (5, 5, 5), (1, 1, 3)])
@pytest.mark.parametrize("dataflow", [0, 1, 2])
def test_downsampling_maps(dev, scene_small, bits, ksize, dataflow):
    rk, tk = _keys(scene_small, bits, dev)
    ts = (1, 1, 2) if ksize == (1, 1, 3) else (2, 2, 2)
    rt = orc.downsample(rk, ts)
    tt = torch.from_numpy(rt).to(dev)
    got = F.build_kmap(tk, tt, ksize, 1, dataflow)
    ref = orc.build_kmap(rk, rt, ksize, (1, 1, 1), dataflow)
    assert_tuple_equal(got, ref, f"bits={bits} k={ksize} dataflow={dataflow}")


def test_strided_source_maps(dev, scene_small):
    # stride-2 sources (a deeper U-Net level) with k=3 and k=2 maps
    rk, _ = _keys(scene_small, 64, dev)
    s2 = orc.downsample(rk, (2, 2, 2))
    s4 = orc.downsample(rk, (4, 4, 4))
    t2, t4 = torch.from_numpy(s2).to(dev), torch.from_numpy(s4).to(dev)
    for d in (0, 1, 2):
        assert_tuple_equal(F.build_kmap(t2, t2, 3, 2, d), orc.build_kmap(s2, s2, (3, 3, 3), (2, 2, 2), d), "s2 k3")
        assert_tuple_equal(F.build_kmap(t2, t4, 2, 2, d), orc.build_kmap(s2, s4, (2, 2, 2), (2, 2, 2), d), "s2 k2")


@pytest.mark.parametrize("ksize", [3, 5])
def test_no_small_z(dev, scene_small, ksize):
    rk, tk = _keys(scene_small, 64, dev)
    got = F.build_kmap_no_small_z(tk, tk, ksize, 1)
    ref = orc.build_kmap_no_small_z(rk, rk, (ksize,) * 3, (1, 1, 1))
    assert_tuple_equal(got, ref, "no_small_z")


def test_convert_transposed(dev, scene_small):
    rk, tk = _keys(scene_small, 64, dev)
    rt = orc.downsample(rk, (2, 2, 2))
    tt = torch.from_numpy(rt).to(dev)
    m = F.build_kmap(tk, tt, 2, 1, 0)
    got = F.convert_transposed_os(m[2], m[0])
    assert np.array_equal(np_(got), orc.convert_transposed_os(np_(m[2]), m[0]))


@pytest.mark.parametrize("ksize,stride", [(3, 1), (5, 1), (3, 2), (5, 2)])
def test_lidar_config2_maps(dev, scene_lidar, ksize, stride):
    """Config 2: the ~100k-voxel LiDAR scene, k in {3,5}, stride in {1,2}."""
    rk, tk = _keys(scene_lidar, 64, dev)
    if stride == 1:
        rt, tt = rk, tk
    else:
        rt = orc.downsample(rk, (2, 2, 2))
        tt = torch.from_numpy(rt).to(dev)
    got = F.build_kmap(tk, tt, ksize, 1, 0)
    ref = orc.build_kmap(rk, rt, (ksize,) * 3, (1, 1, 1), 0)
    assert_tuple_equal(got, ref, f"lidar k={ksize} s={stride}")
    got = F.build_kmap(tk, tt, ksize, 1, 1)
    ref = orc.build_kmap(rk, rt, (ksize,) * 3, (1, 1, 1), 1)
    assert_tuple_equal(got, ref, f"lidar ws k={ksize} s={stride}")


def test_edge_cases(dev):
    # single voxel, coordinates at zero (negative offsets wrap), voxel at the
    # top of the 32-bit z range, a target absent from the sources, T not a
    # multiple of 64 / 128
    pts = np.array([[0, 0, 0], [0, 0, 1], [1, 0, 0], [0, 1, 255], [4095, 4095, 255], [7, 7, 7]], np.int32)
    for bits in (32, 64):
        for n in (1, 2, len(pts)):
            rk, tk = _keys(pts[:n], bits, dev)
            for d in range(9):
                got = F.build_kmap(tk, tk, 3, 1, d)
                assert_tuple_equal(got, orc.build_kmap(rk, rk, (3, 3, 3), (1, 1, 1), d), f"edge n={n} d={d}")
    # targets that are not sources
    rk, tk = _keys(pts[:3], 64, dev)
    rt, tt = _keys(pts[3:], 64, dev)
    for d in (0, 1, 2):
        assert_tuple_equal(F.build_kmap(tk, tt, 3, 1, d), orc.build_kmap(rk, rt, (3, 3, 3), (1, 1, 1), d), "disjoint")


def test_wide_window_fallback(dev):
    """Sparse targets over dense sources: the per-wave source window exceeds
    the LDS cap and the global-memory search path runs."""
    g = np.stack(np.meshgrid(np.arange(64), np.arange(64), np.arange(16), indexing="ij"), -1).reshape(-1, 3)
    src = g.astype(np.int32)
    tgt = g[::97].astype(np.int32)
    rk, tk = _keys(src, 64, dev)
    rt, tt = _keys(tgt, 64, dev)
    for d in (0, 1, 2):
        got = F.build_kmap(tk, tt, 3, 1, d)
        assert_tuple_equal(got, orc.build_kmap(rk, rt, (3, 3, 3), (1, 1, 1), d), f"wide d={d}")


@pytest.mark.parametrize("concurrent", [False, True])
def test_streamed_build_matches_single(dev, scene_small, concurrent):
    """Network-wide build (UNet layer list) equals per-layer builds, also
    with every map on a side stream of its own (the opt-in fan-out)."""
    from spira_amd.nn.functional import _native
    rk, tk = _keys(scene_small, 64, dev)
    _native._C.set_concurrent_maps(concurrent)
    try:
        _check_streamed(tk)
    finally:
        _native._C.set_concurrent_maps(False)


def _check_streamed(tk):
    target_strides = [(2, 2, 2), (4, 4, 4), (8, 8, 8), (16, 16, 16)]
    voxels = [tk] + list(F.streamed_output_generate(tk, target_strides))
    ks = [(3, 3, 3), (2, 2, 2)] * 4 + [(3, 3, 3)]
    ss = [(1, 1, 1), (1, 1, 1), (2, 2, 2), (2, 2, 2), (4, 4, 4), (4, 4, 4), (8, 8, 8), (8, 8, 8), (16, 16, 16)]
    # the hybrids (5-8) on the submanifold maps transpose their dense part
    # after the side stream that built the map has finished
    for dfs in ([0] * 9, [1] * 9, [2] * 9, [0, 1, 2, 0, 1, 2, 0, 1, 2], [6, 0, 8, 0, 5, 0, 7, 0, 6],
                [3, 1, 4, 2, 3, 1, 4, 2, 3]):
        maps = F.build_kmap_streamed(voxels, ks, ss, dfs)
        for i, m in enumerate(maps):
            src, tgt = np_(voxels[i // 2]), np_(voxels[(i + 1) // 2])
            half = (i % 2 == 0) if dfs[i] == 2 else None
            ref = orc.build_kmap(src, tgt, ks[i], ss[i], dfs[i], half=half)
            assert_tuple_equal(m, ref, f"streamed map {i} dataflow {dfs[i]}")


@pytest.mark.parametrize("prepare", [True, False])
@pytest.mark.parametrize("df", [0, 1, 2])
def test_network_wide_cache_build(dev, prepare, df):
    """KernelMapCache.add_all_kernel_maps (output-stationary maps on the
    current stream, the other dataflows on one pool stream each, row orders
    queued with the build) caches, for every layer, the map the oracle builds
    for that layer's voxel sets; a row order queued at build time is the one
    a layer would compute itself."""
    import spira_amd
    from spira_amd.networks import kmap_schedule
    from spira_amd.nn.functional import _native
    coords = scenes.indoor(target=120_000, seed=3)
    rk, _ = orc.flatten_sort(coords, True)
    cache = spira_amd.nn.KernelMapCache()
    cache.prepare_row_orders = prepare
    x = spira_amd.SparseTensor(coordinates=torch.from_numpy(coords).to(dev),
                               features=torch.zeros(len(coords), 3, device=dev).half(), double=True)
    x.order()
    ts, ks, ss = kmap_schedule("UNet")
    cache.add_all_kernel_maps(x._coordinates, ks, ss, ts, (1, 1, 1), [df] * len(ks))
    vox = {(1, 1, 1): rk}
    for t in ts:
        vox[t] = orc.downsample(rk, t)
        assert np.array_equal(np_(cache._coordinates_cache[t]), vox[t]), f"coordinates at stride {t}"
    for i, k in enumerate(ks):
        s_src, s_tgt = ss[i], ss[i + 1]
        entry = cache._kernel_maps_cache[(s_src, s_tgt, k)]
        half = (i % 2 == 0) if df == 2 else None
        ref = orc.build_kmap(vox[s_src], vox[s_tgt], k, s_src, df, half=half)
        assert_tuple_equal(tuple(entry[1:]), ref, f"cached map {i} dataflow {df}")
        if df == 0 and entry[2] >= 100_000 and int(np.prod(k)) >= 27:
            m, T = entry[3], entry[2]
            order, masks, omap = _native._C.kmap_row_order(m, T)
            o2, m2, om2 = _native._C.kmap_row_order(m.clone(), T)  # computed afresh
            assert torch.equal(order, o2) and torch.equal(masks, m2) and torch.equal(omap, om2)


@pytest.mark.parametrize("ks", [(2, 2, 2), (1, 2, 2)])
def test_convert_transposed_partition(dev, ks):
    """The one-pass inverse of a down-sampling map whose kernel is its stride
    (every source in exactly one entry) equals the general inverse, padding
    rows included: the config-4 scene and a small ragged one."""
    for c in (scenes.indoor(), scenes.spheres_planes(n=3001, grid=40, seed=2)):
        k, _ = orc.flatten_sort(c, True)
        kd = orc.downsample(k, ks)
        m = orc.build_kmap(k, kd, ks, (1, 1, 1), 0)[2]
        ref = orc.convert_transposed_os(m, len(k))
        md = torch.from_numpy(np.ascontiguousarray(m)).to(dev)
        got = F.convert_transposed_os(md, len(k), partition=True)
        assert np.array_equal(np_(got), ref)
        assert np.array_equal(np_(F.convert_transposed_os(md, len(k))), ref)


@pytest.mark.parametrize("ks", [(2, 2, 2), (1, 2, 2)])
def test_convert_transposed_partition_order(dev, ks):
    """The inverse of a partition map with its row order made in the same
    pass: the inverse equals the oracle's, and the cached order, group masks
    and ordered map equal the general row order of the same inverse (computed
    on a copy, sorted); a transposed fp16 layer walking it matches the oracle."""
    from spira_amd.nn.functional._native import _C
    for c in (scenes.indoor(), scenes.spheres_planes(n=3001, grid=40, seed=2)):
        k, _ = orc.flatten_sort(c, True)
        for s in (1, 2, 4):
            kf = k if s == 1 else orc.downsample(k, (s,) * 3)
            st = tuple(s * q for q in ks)
            kc = orc.downsample(k, st)
            m = orc.build_kmap(kf, kc, ks, (s,) * 3, 0)[2]
            S, T = len(kf), len(kc)
            print(f"[partition order] S={S} T={T} ks={ks} stride={s}", flush=True)
            md = torch.from_numpy(np.ascontiguousarray(m)).to(dev)
            inv = F.convert_transposed_os_ordered(md, T, S)
            assert np.array_equal(np_(inv), orc.convert_transposed_os(m, S))
            got = [np_(t) for t in _C.kmap_row_order(inv, S)]
            ref = [np_(t) for t in _C.kmap_row_order(inv.clone(), S)]
            for g, r in zip(got, ref):
                assert np.array_equal(g, r)
    g = torch.Generator().manual_seed(3)
    X = torch.randn(T, 64, generator=g).half()
    W = (torch.randn(m.shape[1], 64, 48, generator=g) / 20).half()
    invn = orc.convert_transposed_os(m, S)
    y = F.sparse_convolution_forward_os(T, S, inv, X.to(dev), W.to(dev))
    assert rel_err(np_(y.float()), orc.conv_os(invn, S, X.double().numpy(), W.double().numpy())) <= 1e-2


def test_convert_transposed_ordered_not_a_partition(dev):
    """A k = 2 map whose targets are a subset of the down-sampled sources
    leaves some sources in no entry: the inverse made with its row order must
    still be exact (those rows all -1), its order a permutation of the
    sources, and a transposed layer walking it must match the oracle on
    every row (the uncovered rows get a zero sum)."""
    from spira_amd.nn.functional._native import _C
    c = scenes.spheres_planes(n=20000, grid=64, seed=9)
    k, _ = orc.flatten_sort(c, True)
    kc = orc.downsample(k, (2, 2, 2))[::3].copy()     # every third coarse voxel
    m = orc.build_kmap(k, kc, (2, 2, 2), (1, 1, 1), 0)[2]
    S, T = len(k), len(kc)
    assert int((m >= 0).sum()) < S
    print(f"[non-partition inverse] S={S} T={T}", flush=True)
    md = torch.from_numpy(np.ascontiguousarray(m)).to(dev)
    inv = F.convert_transposed_os_ordered(md, T, S)
    ref = orc.convert_transposed_os(m, S)
    assert np.array_equal(np_(inv), ref)
    order, masks, omap = (np_(t) for t in _C.kmap_row_order(inv, S))
    assert np.array_equal(np.sort(order), np.arange(S))
    assert np.array_equal(omap, ref[:S][order])
    g = torch.Generator().manual_seed(4)
    X = torch.randn(T, 32, generator=g).half()
    W = (torch.randn(8, 32, 32, generator=g) / 16).half()
    y = F.sparse_convolution_forward_os(T, S, inv, X.to(dev), W.to(dev))
    assert rel_err(np_(y.float()), orc.conv_os(ref, S, X.double().numpy(), W.double().numpy())) <= 1e-2


def test_downsample_chain_large(dev):
    """An input above 1024 compaction tiles (2.3M keys): the chained
    downsample takes the device-wide scan at every level (the levels are
    sized by the input); every level against the oracle."""
    rng = np.random.default_rng(31)
    c = np.unique(rng.integers(0, 600, size=(2_300_000, 3)), axis=0).astype(np.int32)
    assert len(c) > 2048 * 1024
    rk, _ = orc.flatten_sort(c, True)
    strides = [(2, 2, 2), (4, 4, 4), (8, 8, 8), (16, 16, 16)]
    outs = F.streamed_output_generate(torch.from_numpy(rk).to(dev), strides)
    for o, s in zip(outs, strides):
        assert np.array_equal(np_(o), orc.downsample(rk, s)), s


def test_row_order_batch_matches_single(dev):
    """The row orders of several maps made in one batched chain of launches
    (prepare_row_orders: one sort over all their rows) equal each map's own
    row order (kmap_row_order of a copy), for maps of 27, 8 and 7 offsets (the
    batch takes the 27-offset maps, the others keep their own sort) and
    sizes from 300 to 200k rows; a map listed twice is ordered once."""
    from spira_amd.nn.functional._native import _C
    c = scenes.indoor()
    k, _ = orc.flatten_sort(c, True)
    maps, Ts = [], []
    for s in (1, 2, 4, 8):
        kf = k if s == 1 else orc.downsample(k, (s,) * 3)
        maps.append(torch.from_numpy(orc.build_kmap(kf, kf, (3, 3, 3), (s,) * 3, 0)[2]).to(dev))
        Ts.append(len(kf))
    kd = orc.downsample(k, (2, 2, 2))
    maps.append(torch.from_numpy(orc.build_kmap(k, kd, (2, 2, 2), (1, 1, 1), 0)[2]).to(dev))
    Ts.append(len(kd))
    small = k[:300]
    maps.append(torch.from_numpy(orc.build_kmap(small, small, (1, 1, 7), (1, 1, 1), 0)[2]).to(dev))
    Ts.append(300)
    print(f"[row order batch] T={Ts}", flush=True)
    _C.prepare_row_orders(maps + [maps[0]], Ts + [Ts[0]], [1] * (len(maps) + 1))
    for m, T in zip(maps, Ts):
        got = [np_(t) for t in _C.kmap_row_order(m, T)]
        ref = [np_(t) for t in _C.kmap_row_order(m.clone(), T)]
        for g, r in zip(got, ref):
            assert np.array_equal(g, r), f"T={T} K={m.shape[1]}"
