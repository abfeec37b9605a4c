"""Pins of the CPU oracle (oracle/) against independent formulations.

The reference ships no golden vectors or unit tests for this path (its only
correctness script compares against external engines that are not available
here), so every oracle function is checked against what the mathematics
fixes: numpy closed forms, brute-force dictionary / dense-grid lookups,
set recomputations, inverse-permutation identities and float64 einsums.
"""
import itertools

import numpy as np
import pytest

from oracle import oracle as orc

RNG = np.random.default_rng(2026)


def _kmin(k):
    return -(k // 2) if k % 2 == 1 else -(k // 2) + 1


def _canonical_offsets(ksize):
    kx, ky, kz = ksize
    return [(x, y, z) for x in range(_kmin(kx), _kmin(kx) + kx) for y in range(_kmin(ky), _kmin(ky) + ky)
            for z in range(_kmin(kz), _kmin(kz) + kz)]


def _pack_py(x, y, z, bits):
    xs, ys = (40, 16) if bits == 64 else (20, 8)
    m = (1 << bits) - 1
    return (((x & m) << xs) | ((y & m) << ys) | (z & m)) & m


def _off_py(dx, dy, dz, bits):
    """Packed offset: signed per-axis deltas added (not OR-ed) modulo 2^bits."""
    xs, ys = (40, 16) if bits == 64 else (20, 8)
    return ((dx << xs) + (dy << ys) + dz) & ((1 << bits) - 1)


def _cloud(n, extent, seed=0):
    r = np.random.default_rng(seed)
    c = np.unique(r.integers(0, extent, size=(n, 3)), axis=0).astype(np.int32)
    return c


# ---------------------------------------------------------------- packing

@pytest.mark.parametrize("bits", [32, 64])
def test_pack_matches_closed_form(bits):
    c = RNG.integers(-5, 4000, size=(500, 3)).astype(np.int32)
    got = orc.to_u64(orc.pack(c, bits))
    exp = np.array([_pack_py(int(x), int(y), int(z), bits) for x, y, z in c], dtype=np.uint64)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("bits,ext", [(32, (4096, 4096, 256)), (64, (1 << 24, 1 << 24, 1 << 16))])
def test_unpack_inverts_pack_in_range(bits, ext):
    c = np.stack([RNG.integers(0, e, 1000) for e in ext], axis=1).astype(np.int32)
    assert np.array_equal(orc.unflatten(orc.pack(c, bits)), c)


def test_flatten_sort_is_lexicographic_and_stable():
    c = RNG.integers(0, 50, size=(3000, 3)).astype(np.int32)  # duplicates present
    for double in (False, True):
        keys, perm = orc.flatten_sort(c, double)
        exp = np.lexsort((np.arange(len(c)), c[:, 2], c[:, 1], c[:, 0]))
        assert np.array_equal(perm, exp)
        assert np.all(np.diff(orc.to_u64(keys).astype(np.float64)) >= 0)


@pytest.mark.parametrize("stride", [(2, 2, 2), (4, 4, 4), (1, 1, 2), (8, 2, 16)])
def test_downsample_is_floor_unique(stride):
    c = _cloud(4000, 200)
    for bits in (32, 64):
        keys, _ = orc.flatten_sort(c, bits == 64)
        got = orc.unflatten(orc.downsample(keys, stride))
        exp = np.unique((c // np.array(stride)) * np.array(stride), axis=0)
        assert np.array_equal(got, exp)


# ---------------------------------------------------------------- offsets

def test_offsets_enumeration():
    for ksize, stride in [((3, 3, 3), (1, 1, 1)), ((2, 2, 2), (2, 2, 2)), ((5, 5, 5), (4, 4, 4)), ((1, 1, 3), (8, 8, 8))]:
        for bits in (32, 64):
            full = orc.offsets_full(ksize, stride, bits)
            exp = [_off_py(dx * stride[0], dy * stride[1], dz * stride[2], bits)
                   for dx, dy, dz in _canonical_offsets(ksize)]
            assert [int(v) for v in full] == exp
            xy = orc.offsets(ksize, stride, bits)
            assert [int(v) for v in xy] == exp[::ksize[2]]  # the iz = 0 (z = kz_min) member of each column


@pytest.mark.parametrize("dataflow,front", [(3, 1), (4, 1), (5, 7), (6, 7), (7, 19), (8, 19)])
def test_indexes_l1(dataflow, front):
    perm, nf = orc.indexes_l1((3, 3, 3), dataflow)
    assert nf == front
    assert sorted(perm.tolist()) == list(range(27))
    thr = (dataflow - 1) // 2
    offs = _canonical_offsets((3, 3, 3))
    fronts = [k for k, o in enumerate(offs) if sum(map(abs, o)) < thr]
    backs = [k for k, o in enumerate(offs) if sum(map(abs, o)) >= thr]
    assert [int(perm[k]) for k in fronts] == list(range(front))
    assert [int(perm[k]) for k in backs] == list(range(front, 27))
    # the mirror of the r-th back offset is the (27-front-1-r)-th back offset
    for r, k in enumerate(backs):
        assert backs[len(backs) - 1 - r] == 26 - k


# ---------------------------------------------------------------- search

def _brute_map(src_keys, tgt_keys, ksize, stride, bits):
    """Exact modular lookup of key_t + offset_k in the source key set, with
    the one case where the reference's lower-bound + z-scan differs from an
    exact lookup: once the z-walk c0, c0+sz, ... of a column passes 2^bits
    (c0 wrapped below zero, e.g. voxels at x = y = 0 with negative offsets),
    the scan index sits at or past every source key and the remaining
    entries are -1 (query_sorted.cuh:131-150)."""
    su = [int(v) for v in orc.to_u64(src_keys)]
    where = {k: i for i, k in enumerate(su)}
    m = (1 << bits) - 1
    kz, sz = ksize[2], stride[2]
    offs = [_off_py(dx * stride[0], dy * stride[1], dz * stride[2], bits) for dx, dy, dz in _canonical_offsets(ksize)]
    T = len(tgt_keys)
    Tp = orc.round128(T)
    out = np.full((len(offs), Tp), -1, np.int32)
    for t, key in enumerate(orc.to_u64(tgt_keys)):
        for k, o in enumerate(offs):
            iz = k % kz
            c0 = (int(key) + o - iz * sz) & m  # the column's first query
            if c0 + iz * sz > m:
                continue  # the walk wrapped past 2^bits: -1
            out[k, t] = where.get((int(key) + o) & m, -1)
    return out


def test_origin_wrap_case_is_covered():
    """The wrap rule above is exercised: the voxel at the origin loses its
    own centre entry under a 3x3x3 map (c0 = -1 wraps)."""
    c = np.array([[0, 0, 0], [0, 0, 1], [1, 1, 1]], np.int32)
    keys, _ = orc.flatten_sort(c, True)
    ws = orc.search(keys, keys, (3, 3, 3), (1, 1, 1), orc.WS)
    assert ws[13, 0] == -1  # centre of (0,0,0): the z-walk started at 2^64-1
    assert ws[13, 1] == 1   # centre of (0,0,1): c0 = (0,0,0) does not wrap
    assert np.array_equal(ws, _brute_map(keys, keys, (3, 3, 3), (1, 1, 1), 64))


@pytest.mark.parametrize("bits", [32, 64])
@pytest.mark.parametrize("ksize", [(3, 3, 3), (2, 2, 2), (5, 5, 5), (1, 1, 3)])
def test_search_equals_exact_lookup(bits, ksize):
    c = _cloud(1500, 14, seed=1)  # includes zeros: negative offsets wrap
    keys, _ = orc.flatten_sort(c, bits == 64)
    ws = orc.search(keys, keys, ksize, (1, 1, 1), orc.WS)
    assert np.array_equal(ws, _brute_map(keys, keys, ksize, (1, 1, 1), bits))


def test_search_downsampled_targets_and_strided_sources():
    c = _cloud(2000, 30, seed=2)
    keys, _ = orc.flatten_sort(c, True)
    t2 = orc.downsample(keys, (2, 2, 2))
    ws = orc.search(keys, t2, (2, 2, 2), (1, 1, 1), orc.WS)
    assert np.array_equal(ws, _brute_map(keys, t2, (2, 2, 2), (1, 1, 1), 64))
    t4 = orc.downsample(keys, (4, 4, 4))
    ws = orc.search(t2, t4, (3, 3, 3), (2, 2, 2), orc.WS)
    assert np.array_equal(ws, _brute_map(t2, t4, (3, 3, 3), (2, 2, 2), 64))


def test_search_dense_grid_neighbours():
    """On a full grid every interior voxel has all 27 neighbours, and the
    entry is the row of the neighbouring coordinate."""
    # shifted off the origin so that no z-walk wraps past 2^64 (see _brute_map)
    g = 1 + np.stack(np.meshgrid(*(np.arange(6),) * 3, indexing="ij"), -1).reshape(-1, 3).astype(np.int32)
    keys, perm = orc.flatten_sort(g, True)
    coords = orc.unflatten(keys)
    index = {tuple(c): i for i, c in enumerate(coords)}
    ws = orc.search(keys, keys, (3, 3, 3), (1, 1, 1), orc.WS)
    for t, c in enumerate(coords):
        for k, (dx, dy, dz) in enumerate(_canonical_offsets((3, 3, 3))):
            nb = (c[0] + dx, c[1] + dy, c[2] + dz)
            assert ws[k, t] == index.get(nb, -1)


def test_layouts_are_permutations_of_each_other():
    c = 1 + _cloud(800, 12, seed=3)  # off the origin: the centre row is then the identity
    keys, _ = orc.flatten_sort(c, True)
    ws = orc.search(keys, keys, (3, 3, 3), (1, 1, 1), orc.WS)
    os_ = orc.search(keys, keys, (3, 3, 3), (1, 1, 1), orc.OS)
    noz = orc.search(keys, keys, (3, 3, 3), (1, 1, 1), orc.NOZ)
    assert np.array_equal(noz, ws.T)
    # z-major: column iz*O + o holds canonical row o*kz + iz
    zmaj = [o * 3 + iz for iz in range(3) for o in range(9)]
    assert np.array_equal(os_, ws.T[:, zmaj])
    perm, _ = orc.indexes_l1((3, 3, 3), 7)
    hy = orc.search(keys, keys, (3, 3, 3), (1, 1, 1), orc.HYBRID, perm)
    assert np.array_equal(hy[perm], ws)
    # padded targets are -1, the centre is the identity, and the map is symmetric
    T = len(keys)
    assert np.all(ws[:, T:] == -1)
    assert np.array_equal(ws[13, :T], np.arange(T))
    for k in range(27):
        for t in np.nonzero(ws[k, :T] >= 0)[0]:
            assert ws[26 - k, ws[k, t]] == t


# ---------------------------------------------------------------- compaction

def test_ws_pairs_recomputed():
    c = _cloud(900, 12, seed=4)
    keys, _ = orc.flatten_sort(c, True)
    ws = orc.search(keys, keys, (3, 3, 3), (1, 1, 1), orc.WS)
    for row0, R in [(0, 27), (0, 14), (7, 10)]:
        nbmaps, nbs, na, qna, P, QP = orc.ws_pairs(ws, row0, R)
        rows = ws[row0:row0 + R]
        r_idx, t_idx = np.nonzero(rows >= 0)  # row-major order == (row, t) order
        assert np.array_equal(nbmaps[0], rows[r_idx, t_idx])
        assert np.array_equal(nbmaps[1], t_idx)
        assert np.array_equal(nbs, (rows >= 0).sum(1))
        assert np.array_equal(na, np.concatenate([[0], np.cumsum(nbs)]))
        assert np.array_equal(qna, np.concatenate([[0], np.cumsum((nbs + 127) // 128 * 128)]))
        assert P == na[-1] and QP == qna[-1]


@pytest.mark.parametrize("half", [False, True])
def test_gs_masks_recomputed(half):
    c = _cloud(700, 11, seed=5)
    keys, _ = orc.flatten_sort(c, True)
    S = T = len(keys)
    ws = orc.search(keys, keys, (3, 3, 3), (1, 1, 1), orc.WS)
    R = 14 if half else 27
    sm, tm, nbs = orc.gs_masks(ws, S, T, 0, R, 27, half)
    for k in range(27):
        # with half masks, row k >= 14 is derived from row 26-k; either way
        # it must equal the ranks of row k's own entries (map symmetry)
        ts = np.nonzero(ws[k, :T] >= 0)[0]
        src = ws[k, ts]
        if not half or k < 14:
            exp_t = np.full(T, -1, np.int32)
            exp_t[ts] = np.arange(len(ts))
            exp_s = np.full(S, -1, np.int32)
            exp_s[src] = np.arange(len(ts))
            assert np.array_equal(tm[k], exp_t) and np.array_equal(sm[k], exp_s)
        else:
            # mirrored row: pairs of row 26-k with roles swapped, ranked in row 26-k's order
            mt = np.nonzero(ws[26 - k, :T] >= 0)[0]
            ms = ws[26 - k, mt]
            exp_t = np.full(T, -1, np.int32)
            exp_t[ms] = np.arange(len(mt))
            exp_s = np.full(S, -1, np.int32)
            exp_s[mt] = np.arange(len(mt))
            assert np.array_equal(tm[k], exp_t) and np.array_equal(sm[k], exp_s)
    assert np.array_equal(nbs, (ws[:R] >= 0).sum(1))


def test_convert_transposed_is_inverse():
    c = _cloud(900, 16, seed=6)
    keys, _ = orc.flatten_sort(c, True)
    t2 = orc.downsample(keys, (2, 2, 2))
    osm = orc.search(keys, t2, (2, 2, 2), (1, 1, 1), orc.OS)
    inv = orc.convert_transposed_os(osm, len(keys))
    assert inv.shape == (orc.round128(len(keys)), 8)
    assert (inv >= 0).sum() == (osm >= 0).sum()
    for t, k in zip(*np.nonzero(osm >= 0)):
        assert inv[osm[t, k], k] == t


def test_padding_buckets():
    sizes = [10, 10, 12, 100, 0, 5]
    assert orc.padding_buckets(sizes, -1).tolist() == [0, 1, 2, 3, 4, 5, 6]
    assert orc.padding_buckets(sizes, None).tolist() == [0, 6]
    # 10,10 -> 0 redundancy; +12 -> (36-32)/32 = 0.125; +100 -> 2.03; 100+0 -> 1.0; 0+5 -> 1.0
    assert orc.padding_buckets(sizes, 0.2).tolist() == [0, 3, 4, 5, 6]
    # 100+0 -> 1.0 (not above 1.0, merged); +5 -> (300-105)/105 > 1
    assert orc.padding_buckets(sizes, 1.0).tolist() == [0, 3, 5, 6]


# ---------------------------------------------------------------- features

def test_conv_os_matches_einsum():
    T, S, K, ci, co = 50, 40, 7, 5, 6
    m = RNG.integers(-1, S, size=(T + 3, K)).astype(np.int32)
    X = RNG.normal(size=(S, ci))
    W = RNG.normal(size=(K, ci, co))
    G = np.where((m[:T] >= 0)[..., None], X[np.maximum(m[:T], 0)], 0.0)  # [T, K, ci]
    exp = np.einsum("tkc,kcd->td", G, W)
    assert np.allclose(orc.conv_os(m, T, X, W), exp, rtol=0, atol=1e-12)
    assert np.allclose(orc.conv_os_f32(m, T, X, W), exp, rtol=1e-5, atol=1e-5)


def test_conv_pairs_matches_add_at():
    P, S, T, K, ci, co = 300, 30, 20, 4, 3, 5
    ins, outs, w = RNG.integers(0, S, P), RNG.integers(0, T, P), RNG.integers(0, K, P)
    X, W = RNG.normal(size=(S, ci)), RNG.normal(size=(K, ci, co))
    exp = np.zeros((T, co))
    np.add.at(exp, outs, np.einsum("pc,pcd->pd", X[ins], W[w]))
    Y = np.zeros((T, co))
    orc.conv_pairs(ins.astype(np.int32), outs.astype(np.int32), w.astype(np.int32), X, W, Y)
    assert np.allclose(Y, exp, atol=1e-12)


def test_dataflows_agree_in_float64():
    """Every dataflow computes the same convolution once its weight-row order
    is accounted for (z-major for 0, canonical for 1/2, L1 order for 3-8).
    Off the origin: at x = y = 0 the wrapped z-walk drops entries from the
    full map that the mirrored half maps still produce, so there the
    reference's dataflows disagree with each other by construction."""
    c = 1 + _cloud(600, 10, seed=8)
    keys, _ = orc.flatten_sort(c, True)
    S = T = len(keys)
    X = RNG.normal(size=(S, 4))
    Wc = RNG.normal(size=(27, 4, 3))
    ws = orc.search(keys, keys, (3, 3, 3), (1, 1, 1), orc.WS)
    full = orc.conv_os(np.ascontiguousarray(ws.T), T, X, Wc)
    zmaj = [o * 3 + iz for iz in range(3) for o in range(9)]
    m0 = orc.build_kmap(keys, keys, (3, 3, 3), (1, 1, 1), 0)
    assert np.allclose(orc.conv_os(m0[2], T, X, Wc[zmaj]), full, atol=1e-12)
    m1 = orc.build_kmap(keys, keys, (3, 3, 3), (1, 1, 1), 1)
    assert np.allclose(orc.conv_ws_merged(S, T, X, Wc, m1[5], m1[3]), full, atol=1e-12)
    m2 = orc.build_kmap(keys, keys, (3, 3, 3), (1, 1, 1), 2)
    assert np.allclose(orc.conv_ws_gs(S, T, X, Wc, m2[3], m2[4]), full, atol=1e-12)
    for d in range(3, 9):
        perm, _ = orc.indexes_l1((3, 3, 3), d)
        dense = int(perm[0])
        Wh = np.empty_like(Wc)
        Wh[perm] = Wc  # row perm[k] holds canonical offset k
        m = orc.build_kmap(keys, keys, (3, 3, 3), (1, 1, 1), d)
        if d in (3, 4):
            y = X @ Wh[0]
        else:
            y = orc.conv_os(m[2], T, X, Wh[:dense])
        if d % 2 == 1:
            y = orc.conv_ws_merged(S, T, X, Wh, m[5], m[3], woffset=dense, hybrid=True, Y=y)
        else:
            y = orc.conv_ws_gs(S, T, X, Wh, m[3], m[4], woffset=dense, Y=y)
        assert np.allclose(y, full, atol=1e-12), d


# ---------------------------------------------------------------- voxelization

def test_ravel_hash_matches_python_integers():
    """Hash of negative coordinates: int32 -> uint64 sign extension and
    products modulo 2^64, computed here with unbounded Python integers."""
    r = np.random.default_rng(11)
    c = np.concatenate([r.integers(-2**31, 2**31, size=(200, 3)),
                        [[-1, -1, -1], [0, 0, 0], [2**31 - 1, -2**31, 5]]]).astype(np.int32)
    h = orc.ravel_hash(c)
    m = (1 << 64) - 1
    for row, got in zip(c.tolist(), h.tolist()):
        x, y, z = (v & m for v in row)
        assert got == ((x * 73856093) & m) ^ ((y * 19349663) & m) ^ ((z * 83492791) & m)


def _quantize_py(pts, vs):
    """Brute force with Python integers: walk the points in order, keep the
    first voxel of every hash value, sort the kept voxels as tuples."""
    import math
    m = (1 << 64) - 1
    kept = {}
    for row in pts.tolist():
        v = tuple(math.floor(float(p) / s) for p, s in zip(row, vs))
        x, y, z = (a & m for a in v)
        h = ((x * 73856093) & m) ^ ((y * 19349663) & m) ^ ((z * 83492791) & m)
        kept.setdefault(h, v)
    return sorted(kept.values())


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
def test_sparse_quantize_matches_brute_force(dtype):
    """Small signed coordinates collide under this hash often (about one
    voxel in seven here), so the collision rule is exercised, not just the
    sorted floor set."""
    r = np.random.default_rng(12)
    pts = r.uniform(-7.5, 7.5, size=(3000, 3)).astype(dtype)
    vs = (0.5, 0.75, 1.25)
    got = orc.sparse_quantize(pts, vs)
    assert got.dtype == np.int32 and got.tolist() == [list(t) for t in _quantize_py(pts, vs)]
    floor_set = {tuple(t) for t in np.floor(pts.astype(np.float64) / np.array(vs)).astype(np.int64).tolist()}
    assert len(got) < len(floor_set)  # collisions present


def test_sparse_quantize_without_collisions_is_sorted_floor_set():
    r = np.random.default_rng(13)
    pts = r.uniform(0, 64, size=(2000, 3))
    got = orc.sparse_quantize(pts, 1.0)
    floor_set = sorted({tuple(t) for t in np.floor(pts).astype(np.int64).tolist()})
    assert len(set(orc.ravel_hash(np.array(floor_set, dtype=np.int32)).tolist())) == len(floor_set)
    assert got.tolist() == [list(t) for t in floor_set]


def test_sparse_quantize_scalar_voxel_and_edges():
    assert orc.sparse_quantize(np.zeros((0, 3)), 1.0).shape == (0, 3)
    assert orc.sparse_quantize(np.array([[-0.5, 0.0, 2.0]]), 1.0).tolist() == [[-1, 0, 2]]
    assert orc.sparse_quantize(np.array([[1.0, 1.0, 1.0]]), 0.5).tolist() == [[2, 2, 2]]


def test_sparse_quantize_collision_keeps_first_point():
    """Colliding voxels collapse to the one whose point comes first."""
    pts = np.array([[5, 0, 0], [1, 0, 0], [3, 0, 0], [2, 0, 0]], dtype=np.float64)
    got = orc.sparse_quantize(pts, 1.0, hash_fn=lambda c: (c[:, 0] % 2).astype(np.uint64))
    assert got.tolist() == [[2, 0, 0], [5, 0, 0]]
