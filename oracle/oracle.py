"""CPU oracle for the Spira kernel-map / sparse-convolution path.

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg, always as the checker.  The product path
(``spira_amd``) never imports it.

It drives ``oracle/liboracle.so`` (``spira_oracle.c``, the C restatement) and
uses numpy for the sort / unique steps.  The functions return the same values,
dtypes and tuple layouts as the reference's ``_C`` entry points:

* ``flatten_sort``      -- torch/cuda_arg_sort_coordinates.cu:11-39
* ``unflatten``         -- torch/cuda_arg_sort_coordinates.cu:41-65
* ``downsample``        -- torch/cuda_arg_sort_coordinates.cu:68-105
* ``build_kmap``        -- torch/cuda_sparse_convolution_mapping.cu:211-892
* ``build_kmap_no_small_z`` -- torch/cuda_sparse_convolution_mapping.cu:1647-1690
* ``convert_transposed_os`` -- torch/cuda_sparse_convolution_mapping.cu:1809-1830
* ``sparse_quantize``   -- datasets/helpers.py:8-31 (voxelization front-end)
* ``conv_*``            -- float64 feature sums with each dataflow's semantics
  (cuda/functions/sparse_convolution.cu, kernels/output_stat.cuh, weight_stat.cuh)

Every function is pinned by tests/test_oracle.py against an independent
formulation (brute-force grids, numpy closed forms, set identities).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional, Sequence, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u64p = np.ctypeslib.ndpointer(dtype=np.uint64, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_I64 = ctypes.c_int64
_I = ctypes.c_int

OS, WS, HYBRID, NOZ = 0, 1, 2, 3


def build() -> str:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    L = ctypes.CDLL(_LIB_PATH)
    L.orc_threads.restype = _I
    L.orc_pack.argtypes = [_i32p, _I64, _I, _u64p]
    L.orc_unpack.argtypes = [_u64p, _I64, _I, _i32p]
    L.orc_downsample_mask.argtypes = [_I, _I, _I, _I]
    L.orc_downsample_mask.restype = ctypes.c_uint64
    L.orc_offsets.argtypes = [_I] * 7 + [_u64p]
    L.orc_offsets.restype = _I
    L.orc_offsets_full.argtypes = [_I] * 7 + [_u64p]
    L.orc_offsets_full.restype = _I
    L.orc_indexes_l1.argtypes = [_I, _I, _I, _I, _i32p]
    L.orc_indexes_l1.restype = _I
    L.orc_search.argtypes = [_u64p, _I64, _u64p, _I64, _I64, _I, _I, _I, _I, _I, _I, _I, _I,
                             ctypes.c_void_p, _i32p]
    L.orc_ws_pairs.argtypes = [_i32p, _I64, _I, _I, _I, _i32p, _i32p, _i32p,
                               ctypes.c_void_p, ctypes.c_void_p]
    L.orc_ws_pairs.restype = _I64
    L.orc_gs_masks.argtypes = [_i32p, _I64, _I64, _I64, _I, _I, _I, _I, _i32p, _i32p, _i32p]
    L.orc_convert_transposed_os.argtypes = [_i32p, _I64, _I, _I64, _i32p]
    L.orc_padding_buckets.argtypes = [_I, _i32p, _I, ctypes.c_double, _i32p]
    L.orc_padding_buckets.restype = _I
    L.orc_conv_os.argtypes = [_i32p, _I64, _I, _f64p, _I, _f64p, _I, _f64p]
    L.orc_conv_pairs.argtypes = [_I64, _i32p, _i32p, _i32p, _f64p, _I, _f64p, _I, _f64p]
    L.orc_conv_os_f32.argtypes = [_i32p, _I64, _I, _f32p, _I, _f32p, _I, _f32p]
    _lib = L
    return L


def threads() -> int:
    return int(lib().orc_threads())


# ----------------------------------------------------------------------------
# key containers
# ----------------------------------------------------------------------------

def _bits_of(keys: np.ndarray) -> int:
    if keys.dtype in (np.int64, np.uint64):
        return 64
    if keys.dtype in (np.int32, np.uint32):
        return 32
    raise TypeError(f"unsupported key dtype {keys.dtype}")


def to_u64(keys: np.ndarray) -> np.ndarray:
    """Signed key tensor (int32 / int64 bit patterns) -> uint64 container."""
    keys = np.ascontiguousarray(keys)
    if _bits_of(keys) == 64:
        return keys.view(np.uint64)
    return keys.view(np.uint32).astype(np.uint64)


def from_u64(u: np.ndarray, bits: int) -> np.ndarray:
    if bits == 64:
        return np.ascontiguousarray(u).view(np.int64)
    return u.astype(np.uint32).view(np.int32)


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int32)


def round128(n: int) -> int:
    return (n + 127) // 128 * 128


# ----------------------------------------------------------------------------
# coordinates
# ----------------------------------------------------------------------------

def pack(coords: np.ndarray, bits: int) -> np.ndarray:
    c = _i32(coords).reshape(-1, 3)
    out = np.empty(c.shape[0], np.uint64)
    lib().orc_pack(c, c.shape[0], bits, out)
    return from_u64(out, bits)


def unflatten(keys: np.ndarray) -> np.ndarray:
    u = to_u64(keys)
    out = np.empty((u.shape[0], 3), np.int32)
    lib().orc_unpack(u, u.shape[0], _bits_of(keys), out)
    return out


def flatten_sort(coords: np.ndarray, double: bool) -> Tuple[np.ndarray, np.ndarray]:
    """Pack then stable ascending sort on the unsigned key
    (arg_sort_coodrinates.cu:36-88: radix SortPairs over all key bits)."""
    bits = 64 if double else 32
    keys = pack(coords, bits)
    u = to_u64(keys)
    perm = np.argsort(u, kind="stable").astype(np.int32)
    return from_u64(u[perm], bits), perm


def downsample_mask(bits: int, stride) -> int:
    sx, sy, sz = stride
    return int(lib().orc_downsample_mask(bits, sx, sy, sz))


def downsample(keys: np.ndarray, stride) -> np.ndarray:
    """keys & mask, then sort + unique (cuda_arg_sort_coordinates.cu:68-105)."""
    bits = _bits_of(keys)
    m = np.uint64(downsample_mask(bits, stride))
    u = np.unique(to_u64(keys) & m)
    return from_u64(u, bits)


def ravel_hash(coords: np.ndarray) -> np.ndarray:
    """x*73856093 ^ y*19349663 ^ z*83492791 over the int32 coordinates
    sign-extended to uint64, products modulo 2^64 (datasets/helpers.py:8-12)."""
    u = np.asarray(coords, dtype=np.int32).astype(np.int64).view(np.uint64)
    with np.errstate(over="ignore"):
        return (u[:, 0] * np.uint64(73856093)) ^ (u[:, 1] * np.uint64(19349663)) ^ (u[:, 2] * np.uint64(83492791))


def sparse_quantize(points: np.ndarray, voxel_size=1.0, hash_fn=ravel_hash) -> np.ndarray:
    """floor(points / voxel_size) in float64 cast to int32; the first point of
    every hash value is kept; the kept voxels are sorted by (x, y, z)
    (datasets/helpers.py:14-31).  ``hash_fn`` exists so that tests can force
    hash collisions."""
    v = np.broadcast_to(np.asarray(voxel_size, dtype=np.float64), (3,))
    c = np.floor(np.asarray(points).astype(np.float64) / v).astype(np.int32).reshape(-1, 3)
    _, first = np.unique(hash_fn(c), return_index=True)
    c = c[first]
    return c[np.lexsort((c[:, 2], c[:, 1], c[:, 0]))]


# ----------------------------------------------------------------------------
# kernel maps
# ----------------------------------------------------------------------------

def offsets(ksize, sstride, bits: int) -> np.ndarray:
    out = np.empty(4096, np.uint64)
    n = lib().orc_offsets(*ksize, *sstride, bits, out)
    return out[:n].copy()


def offsets_full(ksize, sstride, bits: int) -> np.ndarray:
    out = np.empty(4096, np.uint64)
    n = lib().orc_offsets_full(*ksize, *sstride, bits, out)
    return out[:n].copy()


def indexes_l1(ksize, dataflow: int) -> Tuple[np.ndarray, int]:
    K = int(np.prod(ksize))
    data = np.empty(K, np.int32)
    front = lib().orc_indexes_l1(*ksize, dataflow, data)
    return data, int(front)


def search(src: np.ndarray, tgt: np.ndarray, ksize, sstride, layout: int,
           perm: Optional[np.ndarray] = None) -> np.ndarray:
    """Raw search kernel output (query_sorted.cuh:8-297)."""
    bits = _bits_of(src)
    su, tu = to_u64(src), to_u64(tgt)
    S, T = su.shape[0], tu.shape[0]
    Tp = round128(T)
    kx, ky, kz = ksize
    if kz > 64:
        raise ValueError("kz too large for the oracle")
    K = kx * ky * kz
    shape = (K, Tp) if layout in (WS, HYBRID) else (Tp, K)
    out = np.empty(shape, np.int32)
    p = None
    if layout == HYBRID:
        perm = _i32(perm)
        p = perm.ctypes.data_as(ctypes.c_void_p)
    lib().orc_search(np.ascontiguousarray(su), S, np.ascontiguousarray(tu), T, Tp, bits,
                     kx, ky, kz, *sstride, layout, p, out)
    return out


def ws_pairs(wsmap: np.ndarray, row0: int, R: int, q: int = 128):
    Tp = wsmap.shape[1]
    nbs = np.empty(R, np.int32)
    na = np.empty(R + 1, np.int32)
    qna = np.empty(R + 1, np.int32)
    P = int(lib().orc_ws_pairs(_i32(wsmap), Tp, row0, R, q, nbs, na, qna, None, None))
    ins = np.empty(P, np.int32)
    outs = np.empty(P, np.int32)
    lib().orc_ws_pairs(_i32(wsmap), Tp, row0, R, q, nbs, na, qna,
                       ins.ctypes.data_as(ctypes.c_void_p), outs.ctypes.data_as(ctypes.c_void_p))
    return np.stack([ins, outs]), nbs, na, qna, P, int(qna[-1])


def gs_masks(wsmap: np.ndarray, S: int, T: int, row0: int, R: int, Km: int, half: bool):
    Tp = wsmap.shape[1]
    sm = np.empty((Km, S), np.int32)
    tm = np.empty((Km, T), np.int32)
    nbs = np.empty(R, np.int32)
    lib().orc_gs_masks(_i32(wsmap), S, T, Tp, row0, R, Km, int(half), sm, tm, nbs)
    return sm, tm, nbs


def build_kmap(src: np.ndarray, tgt: np.ndarray, ksize, sstride, dataflow: int,
               half: Optional[bool] = None):
    """Reference 9-tuple of cuda_binary_search
    (cuda_sparse_convolution_mapping.cu:211-892).  `half` overrides the
    half-map condition (the streamed build uses `i % 2 == 0`, :1129/:1476)."""
    S, T = int(src.shape[0]), int(tgt.shape[0])
    kx, ky, kz = ksize
    K = kx * ky * kz
    if dataflow == 0:
        return (S, T, search(src, tgt, ksize, sstride, OS), None, None, None, None, None, None)
    if dataflow in (1, 2):
        is_half = (S == T and K % 2 == 1) if half is None else (half and K % 2 == 1)
        wsmap = search(src, tgt, ksize, sstride, WS)
        R = (K + 1) // 2 if is_half else K
        if dataflow == 1:
            nbmaps, nbs, na, qna, P, QP = ws_pairs(wsmap, 0, R)
            return (S, T, wsmap, nbmaps, nbs, na, qna, P, QP)
        sm, tm, nbs = gs_masks(wsmap, S, T, 0, R, K, is_half)
        return (S, T, wsmap, sm, tm, nbs, None, None, None)
    # hybrid dataflows 3..8
    perm, dense = indexes_l1(ksize, dataflow)
    dense = int(perm[0])  # the reference takes data[0] (mapping.cu:779, :821)
    hmap = search(src, tgt, ksize, sstride, HYBRID, perm)
    R = (K - dense) // 2
    first = hmap
    if dataflow > 4:
        first = np.ascontiguousarray(hmap[:dense].T)
    if dataflow % 2 == 1:
        nbmaps, nbs, na, qna, P, QP = ws_pairs(hmap, dense, R)
        return (S, T, first, nbmaps, nbs, na, qna, P, QP)
    sm, tm, nbs = gs_masks(hmap, S, T, dense, R, K - dense, True)
    return (S, T, first, sm, tm, nbs, None, None, None)


def build_kmap_no_small_z(src, tgt, ksize, sstride):
    return (int(src.shape[0]), int(tgt.shape[0]), search(src, tgt, ksize, sstride, NOZ),
            None, None, None, None, None, None)


def convert_transposed_os(osmap: np.ndarray, num_sources: int) -> np.ndarray:
    Tp, K = osmap.shape
    Sp = round128(num_sources)
    out = np.empty((Sp, K), np.int32)
    lib().orc_convert_transposed_os(_i32(osmap), Tp, K, Sp, out)
    return out


def padding_buckets(sizes: Sequence[int], threshold: Optional[float]) -> np.ndarray:
    s = _i32(sizes)
    b = np.empty(len(s) + 1, np.int32)
    nb = lib().orc_padding_buckets(len(s), s, 0 if threshold is None else 1,
                                   0.0 if threshold is None else float(threshold), b)
    return b[:nb + 1].copy()


# ----------------------------------------------------------------------------
# feature sums (float64)
# ----------------------------------------------------------------------------

def _f64(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float64)


def conv_os(osmap: np.ndarray, T: int, X: np.ndarray, W: np.ndarray) -> np.ndarray:
    """Y[t] = sum_j X[map[t,j]] @ W[j] (output_stat.cuh semantics)."""
    Kc = osmap.shape[1]
    Cin, Cout = W.shape[1], W.shape[2]
    assert W.shape[0] == Kc
    Y = np.empty((T, Cout), np.float64)
    lib().orc_conv_os(_i32(osmap), T, Kc, _f64(X), Cin, _f64(W), Cout, Y)
    return Y


def conv_os_f32(osmap: np.ndarray, T: int, X: np.ndarray, W: np.ndarray) -> np.ndarray:
    Kc = osmap.shape[1]
    Cin, Cout = W.shape[1], W.shape[2]
    Y = np.empty((T, Cout), np.float32)
    lib().orc_conv_os_f32(_i32(osmap), T, Kc, np.ascontiguousarray(X, np.float32), Cin,
                          np.ascontiguousarray(W, np.float32), Cout, Y)
    return Y


def conv_pairs(ins, outs, widx, X, W, Y) -> np.ndarray:
    Cin, Cout = W.shape[1], W.shape[2]
    lib().orc_conv_pairs(len(ins), _i32(ins), _i32(outs), _i32(widx), _f64(X), Cin,
                         _f64(W), Cout, Y)
    return Y


def conv_ws_merged(S: int, T: int, X, W, naddrs, nbmaps, transpose: bool = False,
                   woffset: int = 0, hybrid: bool = False,
                   Y: Optional[np.ndarray] = None) -> np.ndarray:
    """Fused weight-stationary semantics (weight_stat.cuh:33-160 driven by
    sparse_convolution.cu:16-60, 1267-1295): pairs of compacted row r use
    W[woffset + r].  The mirrored pass (S == T with an odd kernel volume, or
    any hybrid map) adds X[out] @ W[woffset + Kw-1-r] into Y[in] for every row
    except a self-mirrored centre (2r+1 == Kw), Kw = K - woffset.
    `transpose` swaps the two rows of nbmaps
    (cuda_sparse_convolution_forward.cu:217-226)."""
    K = W.shape[0]
    Cout = W.shape[2]
    if Y is None:
        Y = np.zeros((T, Cout), np.float64)
    ins, outs = (nbmaps[1], nbmaps[0]) if transpose else (nbmaps[0], nbmaps[1])
    ins, outs = _i32(ins), _i32(outs)
    R = len(naddrs) - 1
    Kw = K - woffset
    widx = np.empty(len(ins), np.int32)
    for r in range(R):
        widx[naddrs[r]:naddrs[r + 1]] = woffset + r
    conv_pairs(ins, outs, widx, X, W, Y)
    mirror = hybrid or (S == T and K % 2 == 1)
    if mirror:
        keep = np.ones(len(ins), bool)
        mw = np.empty(len(ins), np.int32)
        for r in range(R):
            mw[naddrs[r]:naddrs[r + 1]] = woffset + (Kw - 1 - r)
            if 2 * r + 1 == Kw:
                keep[naddrs[r]:naddrs[r + 1]] = False
        conv_pairs(outs[keep], ins[keep], mw[keep], X, W, Y)
    return Y


def conv_ws_gs(S: int, T: int, X, W, source_masks, target_masks, woffset: int = 0,
               Y: Optional[np.ndarray] = None) -> np.ndarray:
    """Gather -> GEMM -> scatter semantics (sparse_convolution.cu:1002-1124):
    Y[t] = sum_k X[s] @ W[k] over (s, t) with source_masks[k,s] ==
    target_masks[k,t] >= 0."""
    Km = source_masks.shape[0]
    Cout = W.shape[2]
    if Y is None:
        Y = np.zeros((T, Cout), np.float64)
    ins_l, outs_l, w_l = [], [], []
    for k in range(Km):
        sm = source_masks[k]
        tm = target_masks[k]
        svalid = np.nonzero(sm >= 0)[0]
        n = int(sm.max()) + 1 if svalid.size else 0
        row = np.full(max(n, 1), -1, np.int64)
        row[sm[svalid]] = svalid
        tvalid = np.nonzero(tm >= 0)[0]
        ins_l.append(row[tm[tvalid]].astype(np.int32))
        outs_l.append(tvalid.astype(np.int32))
        w_l.append(np.full(tvalid.size, woffset + k, np.int32))
    if ins_l:
        conv_pairs(np.concatenate(ins_l), np.concatenate(outs_l), np.concatenate(w_l), X, W, Y)
    return Y
