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


def compute_signatures(residual, jl_matrix):
    """Signs of P e for one residual e [d] (python/polarquant_kv/qjl.py:25-35),
    in float64 on the host like the reference's CPU API: QJLSignatures with
    signs = (P e >= 0) and the residual norm."""
    from .types import QJLSignatures
    P = np.asarray(jl_matrix, np.float64)
    e = np.asarray(residual, np.float64)
    return QJLSignatures(signs=(P @ e) >= 0, jl_dim=P.shape[0], residual_norm=float(np.linalg.norm(e)))


def compute_correction(query, signatures, jl_matrix) -> float:
    """(1/m) sum_i (2 s_i - 1) (P q)_i, 0 for a zero residual
    (python/polarquant_kv/qjl.py:38-57). Host float64, as the reference."""
    if signatures.residual_norm < 1e-30:
        return 0.0
    P = np.asarray(jl_matrix, np.float64)
    sv = 2.0 * np.asarray(signatures.signs, np.float64) - 1.0
    return float(np.dot(sv, P @ np.asarray(query, np.float64)) / signatures.jl_dim)


def compute_signatures_gpu(residual, jl_matrix):
    """Device version (src/polarquant_kv_cuda/qjl_kernel.py:6-37): residual
    [..., d] on the GPU, jl_matrix [m, d] -> (packed signs [..., ceil(m/8)]
    uint8 LSB-first, residual norms [...] fp16), by pqkv_qjl_sketch (P e
    summed in fp64; the reference's fp32 product agrees up to projections
    within rounding of 0)."""
    import torch

    from . import _lib
    _lib.require_device(residual)
    P = jl_matrix if isinstance(jl_matrix, torch.Tensor) else torch.from_numpy(np.asarray(jl_matrix))
    P = P.to(device=residual.device, dtype=torch.float64)
    m, d = P.shape
    if residual.shape[-1] != d:
        raise ValueError(f"residual dim {residual.shape[-1]} != JL matrix dim {d}")
    e = residual if residual.dtype in (torch.float16, torch.float32, torch.bfloat16) else residual.float()
    e = e.contiguous()
    lead = e.shape[:-1]
    n = e.numel() // d
    signs = torch.empty(*lead, (m + 7) // 8, dtype=torch.uint8, device=e.device)
    norms = torch.empty(*lead, dtype=torch.float16, device=e.device)
    code = {torch.float16: _lib.F16, torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}[e.dtype]
    _lib.check(_lib.lib().pqkv_qjl_sketch(e.data_ptr(), code, None, P.t().contiguous().data_ptr(), n, d, m,
                                          signs.data_ptr(), norms.data_ptr(), _lib.F16, _lib.stream_of(e)))
    return signs, norms


def compute_correction_gpu(query, packed_signs, residual_norms, jl_matrix):
    """Device version of the correction (src/polarquant_kv_cuda/qjl_kernel.py:40-70):
    query [..., d] against packed signs [..., m/8] of the same leading shape
    -> [...] = (1/m) sum_i (2 s_i - 1) (P q)_i, and 0 where the residual norm
    is 0 (the CPU guard of python/polarquant_kv/qjl.py:50-51, the reference's
    AC-3.5; the reference's device function leaves the norms unread).
    residual_norms None: an all-ones sketch (what a zero residual gives) is
    read as a zero residual."""
    import torch

    from .rotation import rotate
    P = jl_matrix if isinstance(jl_matrix, torch.Tensor) else torch.from_numpy(np.asarray(jl_matrix, np.float32))
    P = P.to(device=query.device, dtype=torch.float32)
    m = P.shape[0]
    bits = bit_unpack(packed_signs, m)
    s = bits.to(torch.float32) * 2.0 - 1.0
    qp = rotate(query.to(torch.float32).contiguous(), P)
    corr = (s * qp).sum(-1) / m
    zero = bits.all(-1) if residual_norms is None else residual_norms.to(corr.device).float() <= 1e-30
    return torch.where(zero, torch.zeros_like(corr), corr)
