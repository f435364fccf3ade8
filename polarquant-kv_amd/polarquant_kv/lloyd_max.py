"""Lloyd-Max codebooks for a rotated unit-vector coordinate.

Mirrors src/polarquant_kv_cuda/lloyd_max.py:12-104 of the reference: the same
names, arguments and return values. The iteration itself must be the
reference's (Beta((d-1)/2,(d-1)/2) on a 50 000-point grid over +-6/sqrt(d),
uniform start, 300 midpoint/centroid updates) for the float32 centroids to
come out identical; unlike the reference the result is cached per
(dim, n_bits, n_iterations, grid_size).
"""

from __future__ import annotations

from functools import lru_cache

import numpy as np


@lru_cache(maxsize=None)
def _codebook(dim: int, n_bits: int, n_iterations: int, grid_size: int):
    from scipy.stats import beta as beta_dist

    levels = 1 << n_bits
    a = (dim - 1) / 2.0
    half_width = 6.0 / np.sqrt(dim)
    grid = np.linspace(-half_width, half_width, grid_size)
    density = beta_dist.pdf(np.clip((grid + 1) / 2, 1e-10, 1 - 1e-10), a, a) / 2
    density = density / (density.sum() * (grid[1] - grid[0]))
    cent = np.linspace(-half_width, half_width, levels)
    edges = np.zeros(levels + 1)
    for _ in range(n_iterations):
        edges = np.empty(levels + 1)
        edges[0], edges[-1] = -2 * half_width, 2 * half_width
        edges[1:-1] = [(cent[i - 1] + cent[i]) / 2 for i in range(1, levels)]
        nxt = cent.copy()
        for i in range(levels):
            sel = (grid >= edges[i]) & (grid < edges[i + 1])
            if sel.sum() > 0:
                w = density[sel]
                total = w.sum()
                if total > 0:
                    nxt[i] = (grid[sel] * w).sum() / total
        cent = nxt
    c = cent.astype(np.float32)
    b = edges.astype(np.float32)
    c.setflags(write=False)
    b.setflags(write=False)
    return c, b


def build_lloyd_max_codebook(dim: int, n_bits: int, n_iterations: int = 300,
                             grid_size: int = 50000) -> tuple[np.ndarray, np.ndarray]:
    """(centroids f32[2^n_bits], boundaries f32[2^n_bits + 1]).

    The boundaries are those of the last iteration's input centroids, as in
    the reference (lloyd_max.py:57-61 vs :77)."""
    if dim < 2 or not 1 <= n_bits <= 8:
        raise ValueError(f"dim must be >= 2 and n_bits in [1, 8], got {dim}, {n_bits}")
    c, b = _codebook(int(dim), int(n_bits), int(n_iterations), int(grid_size))
    return c.copy(), b.copy()


def quantize_with_codebook(values: np.ndarray, centroids: np.ndarray) -> np.ndarray:
    """Index of the nearest centroid, first one on ties (lloyd_max.py:82-90)."""
    return np.abs(np.asarray(values)[..., None] - centroids).argmin(axis=-1).astype(np.uint8)


def dequantize_with_codebook(indices: np.ndarray, centroids: np.ndarray) -> np.ndarray:
    """centroids[indices] (lloyd_max.py:93-98)."""
    return np.asarray(centroids)[indices]


def get_codebook_torch(dim: int, n_bits: int, device="cuda"):
    """Centroids as a float32 torch tensor on `device` (lloyd_max.py:101-104)."""
    import torch

    c, _ = build_lloyd_max_codebook(dim, n_bits)
    return torch.from_numpy(c.copy()).float().to(device)


def padded_codebook_torch(dim: int, n_bits: int, device="cuda"):
    """Centroids padded to 16 float32 entries (the kernels' table width).

    One read-only tensor per (dim, n_bits, device): key and value caches of
    the same width then pass the same codebook pointer, which lets the decode
    kernel serve both from one LDS table. Do not modify it in place."""
    import torch

    return _padded_codebook_dev(dim, n_bits, str(torch.device(device)))


@lru_cache(maxsize=None)
def _padded_codebook_dev(dim: int, n_bits: int, device: str):
    import torch

    c, _ = build_lloyd_max_codebook(dim, n_bits)
    out = np.zeros(16, np.float32)
    out[: c.shape[0]] = c
    return torch.from_numpy(out).to(device)


def stacked_codebooks_torch(dim: int, n_bits: tuple, device="cuda"):
    """padded_codebook_torch for each head width, stacked [H, 16]; shared and
    read-only in the same way."""
    import torch

    return _stacked_codebooks_dev(dim, tuple(int(b) for b in n_bits), str(torch.device(device)))


@lru_cache(maxsize=None)
def _stacked_codebooks_dev(dim: int, n_bits: tuple, device: str):
    import torch

    return torch.stack([_padded_codebook_dev(dim, b, device) for b in n_bits])
