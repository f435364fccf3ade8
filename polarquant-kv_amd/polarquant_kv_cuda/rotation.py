"""Rotation matrix and rotations (src/polarquant_kv_cuda/rotation.py:8-29):
the Haar matrix of scipy's ortho_group from numpy's default_rng(seed) as
fp32 on the device; rotate = v R^T and inverse_rotate = v R on the HIP
rotate kernel for device tensors."""

from __future__ import annotations

from polarquant_kv.rotation import generate_rotation_matrix as _generate
from polarquant_kv.rotation import inverse_rotate, rotate  # noqa: F401


def generate_rotation_matrix(d: int, seed: int | None = None, device="cuda"):
    """d x d orthogonal matrix, float32 on `device` (the reference's default
    device is "cuda")."""
    return _generate(d, seed=seed, device=device)
