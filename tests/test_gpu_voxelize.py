"""GPU voxelization front-end (sparse_quantize, datasets/helpers.py:14-31)
against the oracle: bit-exact int32 voxels, including the hash-collision rule
(the first point of each hash value wins), negative coordinates, float32 and
float64 points, anisotropic voxel sizes and empty / single-point inputs."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from spira_amd.nn import functional as F

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
@pytest.mark.parametrize("n,extent,vs", [(3000, 7.5, (0.5, 0.75, 1.25)), (200000, 40.0, 0.1),
                                          (100000, 3.0, 1.0)])
def test_sparse_quantize_matches_oracle(dev, dtype, n, extent, vs):
    g = torch.Generator().manual_seed(n)
    pts = (torch.rand(n, 3, generator=g, dtype=torch.float64) * 2 - 1) * extent
    pts = pts.to(dtype)
    got = F.sparse_quantize(pts.to(dev), vs)
    want = orc.sparse_quantize(pts.numpy(), vs)
    assert got.dtype == torch.int32 and got.shape == want.shape
    assert np.array_equal(got.cpu().numpy(), want)


def test_sparse_quantize_collisions_present(dev):
    """Inputs where the reference's hash merges distinct voxels."""
    g = torch.Generator().manual_seed(5)
    pts = torch.rand(20000, 3, generator=g, dtype=torch.float64) * 16 - 8
    want = orc.sparse_quantize(pts.numpy(), 0.5)
    distinct = np.unique(np.floor(pts.numpy() / 0.5).astype(np.int32), axis=0)
    assert len(want) < len(distinct)
    assert np.array_equal(F.sparse_quantize(pts.to(dev), 0.5).cpu().numpy(), want)


def test_sparse_quantize_edges(dev):
    assert F.sparse_quantize(torch.zeros(0, 3, device=dev), 1.0).shape == (0, 3)
    one = torch.tensor([[-0.5, 0.0, 2.0]], device=dev)
    assert F.sparse_quantize(one, 1.0).cpu().tolist() == [[-1, 0, 2]]
    same = torch.full((1000, 3), 3.7, dtype=torch.float64, device=dev)
    assert F.sparse_quantize(same, 0.5).cpu().tolist() == [[7, 7, 7]]
    with pytest.raises(Exception):
        F.sparse_quantize(torch.zeros(4, 2, device=dev), 1.0)
    with pytest.raises(Exception):
        F.sparse_quantize(torch.zeros(4, 3, device=dev), 0.0)
