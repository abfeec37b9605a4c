"""The hand-written radix sort (spira_hip_radix_sort_pairs, the sort of
flatten_sort) against numpy's stable argsort, through the C ABI: 64- and
32-bit keys, sizes around the 4096-key tile, duplicates, constant keys (every
pass skipped but one), sorted and reversed input, and the full-range bit
patterns (every pass live)."""
import ctypes
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "spira_amd", "libspira_hip.so")


def _lib():
    lib = ctypes.CDLL(LIB)
    vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.spira_hip_radix_sort_workspace.argtypes = [i64, i32, ctypes.POINTER(ctypes.c_size_t)]
    lib.spira_hip_radix_sort_pairs.argtypes = [vp, vp, vp, vp, i64, i32, vp, ctypes.c_size_t, vp]
    lib.spira_hip_radix_sort_status.argtypes = [vp, i64, i32, vp]
    lib.spira_hip_last_error.restype = ctypes.c_char_p
    return lib


def _sort(lib, keys: np.ndarray, vals: np.ndarray, dev):
    bits = keys.dtype.itemsize * 8
    n = keys.shape[0]
    kd = torch.from_numpy(keys.view(np.int64 if bits == 64 else np.int32)).to(dev)
    vd = torch.from_numpy(vals).to(dev)
    ko, vo = torch.empty_like(kd), torch.full_like(vd, -7)
    wsb = ctypes.c_size_t(0)
    assert lib.spira_hip_radix_sort_workspace(n, bits, ctypes.byref(wsb)) == 0
    ws = torch.empty(max(wsb.value, 1), dtype=torch.uint8, device=dev)
    rc = lib.spira_hip_radix_sort_pairs(kd.data_ptr(), vd.data_ptr(), ko.data_ptr(), vo.data_ptr(), n, bits,
                                        ws.data_ptr(), wsb.value, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, lib.spira_hip_last_error()
    # no tile's look-back wait ran out (else the output would be incomplete)
    rc = lib.spira_hip_radix_sort_status(ws.data_ptr(), n, bits,
                                         ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, lib.spira_hip_last_error()
    torch.cuda.synchronize()
    kin = kd.cpu().numpy().view(keys.dtype)
    assert np.array_equal(kin, keys), "the input keys changed"
    return ko.cpu().numpy().view(keys.dtype), vo.cpu().numpy()


def _check(lib, keys, dev):
    vals = np.arange(keys.shape[0], dtype=np.int32)
    k, v = _sort(lib, keys, vals, dev)
    order = np.argsort(keys, kind="stable")
    assert np.array_equal(k, keys[order])
    assert np.array_equal(v, vals[order])


@pytest.mark.parametrize("dtype", [np.uint64, np.uint32])
@pytest.mark.parametrize("n", [0, 1, 2, 4095, 4096, 4097, 200_000, 1_000_000])
def test_radix_sort_random(dev, dtype, n):
    rng = np.random.default_rng(n + (64 if dtype == np.uint64 else 32))
    full = rng.integers(0, np.iinfo(dtype).max, size=n, dtype=dtype, endpoint=True)
    _check(_lib(), full, dev)


@pytest.mark.parametrize("dtype", [np.uint64, np.uint32])
def test_radix_sort_patterns(dev, dtype):
    lib = _lib()
    rng = np.random.default_rng(7)
    n = 150_000
    few = rng.integers(0, 40, size=n).astype(dtype) << np.asarray(3, dtype=dtype)  # many duplicates
    _check(lib, few, dev)
    _check(lib, np.full(n, 12345, dtype=dtype), dev)  # every digit constant
    s = np.sort(rng.integers(0, 1 << 20, size=n).astype(dtype))
    _check(lib, s, dev)
    _check(lib, s[::-1].copy(), dev)
