"""The allocation-free flatten_sort (spira_hip_flatten_sort_noalloc, its
workspace a fixed device array in the library) against the allocating entry
point spira_hip_flatten_sort, both called through the C ABI: keys and
permutation bit-exact, on two calls in a row (the second smaller, so stale
scratch contents from the first call would show), for 64- and 32-bit keys;
sizes beyond the fixed maximum are rejected with an error."""
import ctypes
import os

import numpy as np
import pytest
import torch

from spira_amd import scenes

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "spira_amd", "libspira_hip.so")
MAX_POINTS = 1 << 20


def _lib():
    lib = ctypes.CDLL(LIB)
    vp, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.spira_hip_flatten_sort_noalloc.argtypes = [vp, i64, i32, vp, vp, vp]
    lib.spira_hip_flatten_sort.argtypes = [vp, i64, i32, vp, vp, vp, ctypes.c_size_t, vp]
    lib.spira_hip_flatten_sort_workspace.argtypes = [i64, i32, ctypes.POINTER(ctypes.c_size_t)]
    lib.spira_hip_last_error.restype = ctypes.c_char_p
    return lib


def _sort_both(lib, coords, bits, dev):
    n = coords.shape[0]
    kd = torch.int64 if bits == 64 else torch.int32
    c = torch.from_numpy(coords).to(dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    # allocating entry point, caller-provided workspace
    wsb = ctypes.c_size_t(0)
    assert lib.spira_hip_flatten_sort_workspace(n, bits, ctypes.byref(wsb)) == 0
    ws = torch.empty(max(wsb.value, 1), dtype=torch.uint8, device=dev)
    k1 = torch.empty(n, dtype=kd, device=dev)
    p1 = torch.empty(n, dtype=torch.int32, device=dev)
    rc = lib.spira_hip_flatten_sort(c.data_ptr(), n, bits, k1.data_ptr(), p1.data_ptr(), ws.data_ptr(), wsb.value,
                                    stream)
    assert rc == 0, lib.spira_hip_last_error()
    # allocation-free entry point; outputs pre-filled with garbage
    k2 = torch.full((n,), -7, dtype=kd, device=dev)
    p2 = torch.full((n,), -7, dtype=torch.int32, device=dev)
    rc = lib.spira_hip_flatten_sort_noalloc(c.data_ptr(), n, bits, k2.data_ptr(), p2.data_ptr(), stream)
    assert rc == 0, lib.spira_hip_last_error()
    torch.cuda.synchronize()
    return k1.cpu(), p1.cpu(), k2.cpu(), p2.cpu()


@pytest.mark.parametrize("bits", [64, 32])
def test_noalloc_matches_allocating_entry_point(dev, bits):
    lib = _lib()
    grid = 2000 if bits == 64 else 250
    big = scenes.spheres_planes(n=300_000 if bits == 64 else 120_000, grid=grid, seed=31)
    small = scenes.spheres_planes(n=5_000, grid=64, seed=32)
    for coords in (big, small):  # second call smaller than the first
        k1, p1, k2, p2 = _sort_both(lib, coords, bits, dev)
        assert torch.equal(k1, k2), f"{bits}-bit keys differ (n={coords.shape[0]})"
        assert torch.equal(p1, p2), f"{bits}-bit permutation differs (n={coords.shape[0]})"
        assert np.all(np.diff(k2.numpy().view(np.uint64 if bits == 64 else np.uint32).astype(np.uint64)) > 0)


def test_noalloc_rejects_oversize(dev):
    lib = _lib()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.spira_hip_flatten_sort_noalloc(None, MAX_POINTS + 1, 64, None, None, stream)
    assert rc != 0
    assert b"1048576" in lib.spira_hip_last_error()


@pytest.mark.parametrize("bits", [64, 32])
def test_noalloc_at_the_maximum(dev, bits):
    """Exactly the documented maximum of 1048576 points (the workspace of
    both key widths fits the fixed scratch), then a smaller call."""
    lib = _lib()
    rng = np.random.default_rng(33 + bits)
    hi = 4000 if bits == 64 else 250
    big = rng.integers(0, hi, size=(MAX_POINTS, 3)).astype(np.int32)
    small = rng.integers(0, hi, size=(777, 3)).astype(np.int32)
    for coords in (big, small):
        k1, p1, k2, p2 = _sort_both(lib, coords, bits, dev)
        assert torch.equal(k1, k2) and torch.equal(p1, p2), f"{bits}-bit, n={coords.shape[0]}"
