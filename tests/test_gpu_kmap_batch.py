"""spira_hip_kmap_search_batch through the C ABI: a batch of output-
stationary searches (3x3x3, 2x2x2 and 5x5x5 maps share launches, other
shapes run alone, more than eight jobs of one shape split over launches, jobs with no
targets) gives every map bit-exact equal to the oracle's search."""
import ctypes
import os

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from spira_amd import scenes

from helpers import np_

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "spira_amd", "libspira_hip.so")


class Job(ctypes.Structure):
    _fields_ = [("sources", ctypes.c_void_p), ("num_sources", ctypes.c_int64), ("targets", ctypes.c_void_p),
                ("num_targets", ctypes.c_int64), ("kx", ctypes.c_int), ("ky", ctypes.c_int), ("kz", ctypes.c_int),
                ("sx", ctypes.c_int), ("sy", ctypes.c_int), ("sz", ctypes.c_int), ("kernel_map", ctypes.c_void_p)]


@pytest.mark.parametrize("bits", [64, 32])
def test_batched_searches(dev, bits):
    lib = ctypes.CDLL(LIB)
    lib.spira_hip_kmap_search_batch.argtypes = [ctypes.c_int, ctypes.POINTER(Job), ctypes.c_int, ctypes.c_void_p]
    lib.spira_hip_last_error.restype = ctypes.c_char_p
    c = scenes.spheres_planes(n=30_000, grid=200 if bits == 64 else 120, seed=7)
    k1, _ = orc.flatten_sort(c, bits == 64)
    levels = {1: k1}
    for s in (2, 4, 8):
        levels[s] = orc.downsample(k1, (s, s, s))
    # (sources stride, targets stride, kernel): submanifold k3, downsampling
    # k2, two k5 and one anisotropic map (unbatched shape), eleven k3 jobs in
    # all (two launches of that shape) and one job without targets
    specs = [(1, 1, 3), (1, 2, 2), (2, 2, 3), (2, 4, 2), (4, 4, 3), (4, 8, 2), (8, 8, 3), (1, 1, 5),
             (2, 2, (1, 1, 3)), (2, 2, 5), (1, 1, 3), (2, 2, 3), (4, 4, 3), (8, 8, 3), (1, 1, 3), (1, 1, 3), (8, 0, 3)]
    dt = torch.int64 if bits == 64 else torch.int32
    keep, jobs, refs = [], [], []
    for ss, ts, k in specs:
        ks = (k, k, k) if isinstance(k, int) else k
        src = levels[ss]
        tgt = levels[ts] if ts else levels[ss][:0]
        sd = torch.from_numpy(src.view(np.int64 if bits == 64 else np.int32)).to(dev)
        td = torch.from_numpy(np.ascontiguousarray(tgt).view(np.int64 if bits == 64 else np.int32)).to(dev)
        Tp = (len(tgt) + 127) // 128 * 128
        m = torch.full((Tp, int(np.prod(ks))), -7, dtype=torch.int32, device=dev)
        keep += [sd, td, m]
        jobs.append(Job(sd.data_ptr(), len(src), td.data_ptr() if len(tgt) else None, len(tgt), *ks,
                        ss, ss, ss, m.data_ptr()))
        refs.append(orc.build_kmap(src, tgt, ks, (ss, ss, ss), 0)[2] if len(tgt) else np.zeros((0, int(np.prod(ks)))))
    arr = (Job * len(jobs))(*jobs)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.spira_hip_kmap_search_batch(len(jobs), arr, bits, stream)
    assert rc == 0, lib.spira_hip_last_error()
    torch.cuda.synchronize()
    for i, ref in enumerate(refs):
        got = np_(keep[3 * i + 2])
        assert got.shape == ref.shape and np.array_equal(got, ref), f"job {i} {specs[i]}"
