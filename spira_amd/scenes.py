"""Seeded synthetic voxel scenes for the benchmark configurations.

Each generator returns unique ``[N, 3] int32`` voxel coordinates, shuffled and
shifted so the per-axis minimum is 0 -- the input convention of the
reference loaders (scripts/loaders.py:6-25).  Voxelisation is floor(p / v)
followed by de-duplication, as in datasets/helpers.py:14-30.
"""
from __future__ import annotations

import numpy as np

__all__ = ["spheres_planes", "lidar", "indoor", "lidar_blobs", "scene_for_config", "voxelize"]

SEED = 2026


def voxelize(points: np.ndarray, voxel: float) -> np.ndarray:
    c = np.floor(points / voxel).astype(np.int64)
    c = np.unique(c, axis=0)
    return c


def _finish(c: np.ndarray, rng: np.random.Generator, n: int | None = None) -> np.ndarray:
    c = np.unique(c, axis=0)
    rng.shuffle(c)
    if n is not None:
        c = c[:n]
    c = c - c.min(axis=0)
    return np.ascontiguousarray(c.astype(np.int32))


def spheres_planes(n: int = 20_000, grid: int = 128, seed: int = SEED) -> np.ndarray:
    """Config 1: points on the surfaces of 8 random spheres and planes inside a
    grid^3 box, voxelised at unit size."""
    rng = np.random.default_rng(seed)
    pts = []
    per = n  # oversample each surface, keep n unique voxels overall
    for i in range(8):
        if i % 2 == 0:  # sphere
            ctr = rng.uniform(0.25 * grid, 0.75 * grid, 3)
            rad = rng.uniform(0.08 * grid, 0.22 * grid)
            v = rng.normal(size=(per, 3))
            v /= np.linalg.norm(v, axis=1, keepdims=True)
            pts.append(ctr + rad * v)
        else:  # plane patch through a random point with a random normal
            p0 = rng.uniform(0.2 * grid, 0.8 * grid, 3)
            nrm = rng.normal(size=3)
            nrm /= np.linalg.norm(nrm)
            a = np.cross(nrm, [1.0, 0.0, 0.0] if abs(nrm[0]) < 0.9 else [0.0, 1.0, 0.0])
            a /= np.linalg.norm(a)
            b = np.cross(nrm, a)
            uv = rng.uniform(-0.3 * grid, 0.3 * grid, (per, 2))
            pts.append(p0 + uv[:, :1] * a + uv[:, 1:] * b)
    p = np.concatenate(pts)
    p = p[np.all((p >= 0) & (p < grid), axis=1)]
    return _finish(np.floor(p).astype(np.int64), rng, n)


def _rings(rng: np.random.Generator, n_rings: int = 64, az_step_deg: float = 0.2, voxel: float = 0.05,
           height: float = 1.8) -> np.ndarray:
    az = np.deg2rad(np.arange(0.0, 360.0, az_step_deg))
    elev = np.deg2rad(np.linspace(-24.8, 2.0, n_rings))
    A, E = np.meshgrid(az, elev)
    A, E = A.ravel(), E.ravel()
    # downward beams hit the ground, the others hit an object at 2-50 m
    ground = np.where(E < 0, height / np.tan(np.maximum(-E, 1e-3)), np.inf)
    obj = rng.uniform(2.0, 50.0, A.size)
    r = np.minimum(ground, obj)
    r = np.clip(r * (1.0 + 0.05 * rng.normal(size=r.size)), 2.0, 50.0)
    x, y = r * np.cos(A), r * np.sin(A)
    z = height + r * np.tan(E)
    return np.stack([x, y, z], axis=1)


def _lidar_points(rng: np.random.Generator, ground_points: int) -> np.ndarray:
    rings = _rings(rng)
    rr = 50.0 * np.sqrt(rng.uniform(0.0, 1.0, ground_points))
    th = rng.uniform(0.0, 2 * np.pi, ground_points)
    g = np.stack([rr * np.cos(th), rr * np.sin(th), np.abs(rng.normal(0.0, 0.02, ground_points))], axis=1)
    return np.concatenate([rings, g])


def _bounded(c: np.ndarray, xy: int = 2048, z: int = 128) -> np.ndarray:
    c = c + np.array([xy // 2, xy // 2, 0])
    keep = (c[:, 0] >= 0) & (c[:, 0] < xy) & (c[:, 1] >= 0) & (c[:, 1] < xy) & (c[:, 2] >= 0) & (c[:, 2] < z)
    return c[keep]


def lidar(target: int = 100_000, seed: int = SEED) -> np.ndarray:
    """Configs 2-3: 64 elevation rings (0.2 deg azimuth step, 2-50 m, 5 %
    range jitter) plus a ground plane, voxelised at 0.05 m into x, y in
    [0, 2048) and z in [0, 128); about `target` unique voxels."""
    rng = np.random.default_rng(seed)
    p = _lidar_points(rng, ground_points=target // 2)
    c = _bounded(voxelize(p, 0.05))
    return _finish(c, rng, target if c.shape[0] > target else None)


def indoor(target: int = 200_000, seed: int = SEED) -> np.ndarray:
    """Config 4: points on 6 walls / floor / ceiling of a 10 m x 10 m x 3 m
    room plus 30 random axis-aligned boxes, voxelised at 2 cm; `target`
    unique voxels."""
    rng = np.random.default_rng(seed)
    L, H, v = 10.0, 3.0, 0.02
    surfaces = []
    # (origin, u-vector, v-vector) of each rectangle
    surfaces += [((0, 0, 0), (L, 0, 0), (0, L, 0)), ((0, 0, H), (L, 0, 0), (0, L, 0)),
                 ((0, 0, 0), (L, 0, 0), (0, 0, H)), ((0, L, 0), (L, 0, 0), (0, 0, H)),
                 ((0, 0, 0), (0, L, 0), (0, 0, H)), ((L, 0, 0), (0, L, 0), (0, 0, H))]
    for _ in range(30):
        size = rng.uniform(0.3, 1.5, 3) * np.array([1.0, 1.0, 1.2])
        o = np.array([rng.uniform(0.2, L - size[0] - 0.2), rng.uniform(0.2, L - size[1] - 0.2), 0.0])
        sx, sy, sz = (np.array([size[0], 0, 0]), np.array([0, size[1], 0]), np.array([0, 0, size[2]]))
        surfaces += [(o, sx, sy), (o + sz, sx, sy), (o, sx, sz), (o + sy, sx, sz), (o, sy, sz), (o + sx, sy, sz)]
    areas = np.array([np.linalg.norm(np.cross(np.array(u, float), np.array(w, float))) for _, u, w in surfaces])
    # sample enough points that ~target unique voxels survive, then subsample
    npts = int(target * 2.2)
    counts = rng.multinomial(npts, areas / areas.sum())
    pts = []
    for (o, u, w), m in zip(surfaces, counts):
        st = rng.uniform(0.0, 1.0, (m, 2))
        pts.append(np.array(o, float) + st[:, :1] * np.array(u, float) + st[:, 1:] * np.array(w, float))
    c = voxelize(np.concatenate(pts), v)
    return _finish(c, rng, target)


def lidar_blobs(target: int = 300_000, seed: int = SEED) -> np.ndarray:
    """Config 5: LiDAR rings plus 50 Gaussian object clusters (sigma 0.5 m),
    voxelised at 0.05 m; about `target` unique voxels."""
    rng = np.random.default_rng(seed)
    p = [_lidar_points(rng, ground_points=target // 3)]
    ctr = np.stack([rng.uniform(-40, 40, 50), rng.uniform(-40, 40, 50), rng.uniform(0.5, 2.5, 50)], axis=1)
    per = (target * 2) // 50
    for cc in ctr:
        p.append(cc + 0.5 * rng.normal(size=(per, 3)))
    c = _bounded(voxelize(np.concatenate(p), 0.05))
    return _finish(c, rng, target if c.shape[0] > target else None)


def scene_for_config(cfg: int, seed: int = SEED) -> np.ndarray:
    if cfg == 1:
        return spheres_planes(seed=seed)
    if cfg in (2, 3):
        return lidar(seed=seed)
    if cfg == 4:
        return indoor(seed=seed)
    if cfg == 5:
        return lidar_blobs(seed=seed)
    raise ValueError(f"unknown config {cfg}")
