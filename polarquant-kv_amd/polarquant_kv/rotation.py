"""Random orthogonal rotation.

Mirrors python/polarquant_kv/rotation.py:7-61 and
src/polarquant_kv_cuda/rotation.py:8-29 of the reference:
generate_rotation_matrix(d, seed) draws a Haar-random R with
scipy.stats.ortho_group from numpy's default_rng(seed) (the distribution and
stream the reference uses, so the same seed gives the same matrix);
rotate(v, R) = v R^T and inverse_rotate(v, R) = v R.

numpy inputs follow the reference's CPU API (float64 arithmetic, result cast
back to the input dtype). torch device tensors go through the HIP rotate
kernel (pqkv_rotate): one fp32 FMA chain per output coordinate.
"""

from __future__ import annotations

import numpy as np

from . import _lib


def generate_rotation_matrix(d: int, seed: int | None = None, device=None):
    """d x d orthogonal matrix; float64 numpy when device is None, else a
    float32 torch tensor on `device` (the two reference variants)."""
    if not isinstance(d, (int, np.integer)):
        raise ValueError(f"d must be an integer, got {type(d).__name__}")
    if d <= 0:
        raise ValueError(f"d must be positive, got {d}")
    if d == 1:
        rng = np.random.Generator(np.random.PCG64(seed))
        R = np.array([[rng.choice([-1.0, 1.0])]], dtype=np.float64)
    else:
        from scipy.stats import ortho_group
        R = ortho_group.rvs(d, random_state=np.random.default_rng(seed)).astype(np.float64)
    if device is None:
        return R
    import torch
    return torch.from_numpy(R).float().to(device)


def _rotate(v, R, inverse: bool):
    if isinstance(v, np.ndarray):
        Rn = np.asarray(R, np.float64)
        return (v.astype(np.float64) @ (Rn if inverse else Rn.T)).astype(v.dtype)
    import torch
    if not isinstance(v, torch.Tensor):
        raise TypeError("v must be a numpy array or a torch tensor")
    _lib.require_device(v, R)
    d = v.shape[-1]
    if R.shape != (d, d):
        raise ValueError(f"R must be ({d}, {d}), got {tuple(R.shape)}")
    x = v.contiguous()
    Rf = R.to(torch.float32).contiguous()
    y = torch.empty_like(x)
    _lib.check(_lib.lib().pqkv_rotate(x.data_ptr(), _lib.dtype_code(x.dtype), Rf.data_ptr(), y.data_ptr(),
                                      _lib.dtype_code(y.dtype), x.numel() // d, d, int(inverse),
                                      _lib.stream_of(x)))
    return y


def rotate(v, rotation_matrix):
    """v @ R^T."""
    return _rotate(v, rotation_matrix, inverse=False)


def inverse_rotate(v, rotation_matrix):
    """v @ R."""
    return _rotate(v, rotation_matrix, inverse=True)
