"""Synthetic sparse-structure inputs for tests and the benchmark.

The reference's sparse stage runs on the active voxels of a decoded occupancy
grid, listed in (batch, x, y, z) lexicographic order
(pipelines/image_to_3d.mojo:108-147). Here a randomly thickened sphere shell
stands in for a decoded shape: voxel p is active when | |p - c| - radius | <=
thickness(p) / 2, with a per-voxel thickness drawn uniformly from
[t_lo, t_hi]. Output: int32 coords [T, 4] sorted (b, x, y, z) and int64
offsets [B + 1].
"""
from __future__ import annotations

import numpy as np


def shell_mask(res: int, radius: float, t_lo: float, t_hi: float, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    ax = np.arange(res, dtype=np.float64)
    c = (res - 1) / 2.0
    d = np.sqrt((ax[:, None, None] - c) ** 2 + (ax[None, :, None] - c) ** 2 + (ax[None, None, :] - c) ** 2)
    thick = rng.uniform(t_lo, t_hi, size=(res, res, res))
    return np.abs(d - radius) <= thick / 2.0


def shell_coords(res: int, batch: int, radius: float, t_lo: float, t_hi: float, seed: int = 0):
    """Ragged batch of `batch` shells on a res^3 grid -> (coords int32 [T, 4], offsets int64 [B+1])."""
    parts, offs = [], [0]
    for b in range(batch):
        m = shell_mask(res, radius, t_lo, t_hi, seed + 7919 * b)
        xyz = np.argwhere(m).astype(np.int32)          # lexicographic (x, y, z)
        cb = np.empty((xyz.shape[0], 4), np.int32)
        cb[:, 0] = b
        cb[:, 1:] = xyz
        parts.append(cb)
        offs.append(offs[-1] + xyz.shape[0])
    coords = np.concatenate(parts, axis=0) if parts else np.zeros((0, 4), np.int32)
    return np.ascontiguousarray(coords), np.asarray(offs, np.int64)


# Config 4: ragged B=2 on 64^3, ~20k voxels each.
C4 = dict(res=64, batch=2, radius=24.0, t_lo=2.0, t_hi=3.5, seed=4)
# Config 5: B=1 on 128^3, ~200k voxels.
C5 = dict(res=128, batch=1, radius=50.0, t_lo=5.0, t_hi=7.8, seed=5)


def config4():
    return shell_coords(**C4)


def config5():
    return shell_coords(**C5)
