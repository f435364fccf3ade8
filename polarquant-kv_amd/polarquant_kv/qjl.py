"""QJL 1-bit sign sketch of the key quantisation residual.

Mirrors python/polarquant_kv/qjl.py:8-57 and
src/polarquant_kv_cuda/qjl_kernel.py:6-135 of the reference:
  P ~ N(0, 1/m), m x d, from numpy PCG64(seed)            (qjl.py:20-21)
  signs = (P e >= 0), packed LSB first, e = k - k_hat     (qjl_kernel.py:26-29,112-124)
  correction(q) = (1/m) sum_i (2 s_i - 1) (P q)_i         (qjl.py:53-55)
On the GPU the sketch is computed at encode time in the rotated space with
P_rot = P R^T (P e = P_rot R e), and the correction is added to the scores
inside the attention kernels.
"""

from __future__ import annotations

import numpy as np


def generate_jl_matrix(jl_dim: int, d: int, seed: int | None = None) -> np.ndarray:
    if jl_dim <= 0:
        raise ValueError(f"jl_dim must be positive, got {jl_dim}")
    rng = np.random.Generator(np.random.PCG64(seed))
    return rng.standard_normal((jl_dim, d)).astype(np.float64) / np.sqrt(jl_dim)


def rotated_jl_matrix(jl_matrix, rotation_matrix, device="cuda"):
    """P_rot = P R^T as a float32 device tensor (the form the kernels use)."""
    import torch

    P = np.asarray(jl_matrix.cpu().numpy() if hasattr(jl_matrix, "cpu") else jl_matrix, np.float64)
    R = np.asarray(rotation_matrix.cpu().numpy() if hasattr(rotation_matrix, "cpu") else rotation_matrix,
                   np.float64)
    return torch.from_numpy((P @ R.T).astype(np.float32)).to(device)


def bit_pack(signs):
    """[..., m] bool -> [..., ceil(m/8)] uint8, bit 0 first (qjl_kernel.py:112-124)."""
    import torch

    m = signs.shape[-1]
    pad = (-m) % 8
    if pad:
        signs = torch.nn.functional.pad(signs, (0, pad))
    g = signs.reshape(*signs.shape[:-1], -1, 8).to(torch.uint8)
    w = torch.tensor([1, 2, 4, 8, 16, 32, 64, 128], dtype=torch.uint8, device=signs.device)
    return (g * w).sum(-1).to(torch.uint8)


def bit_unpack(packed, m: int):
    """Inverse of bit_pack (qjl_kernel.py:127-135)."""
    import torch

    w = torch.tensor([1, 2, 4, 8, 16, 32, 64, 128], dtype=torch.uint8, device=packed.device)
    bits = (packed.unsqueeze(-1) & w) > 0
    return bits.reshape(*packed.shape[:-1], -1)[..., :m]
