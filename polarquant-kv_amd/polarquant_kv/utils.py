"""Helpers of the reference's python/polarquant_kv/utils.py with the same
names and formulas (compression ratio and memory estimates of the group
format, cosine similarity, score MSE)."""

from __future__ import annotations

import math

import numpy as np


def cosine_similarity(a: np.ndarray, b: np.ndarray) -> float:
    """Cosine of two vectors; 0 when either norm is below 1e-30 (utils.py:9-15)."""
    na, nb = np.linalg.norm(a), np.linalg.norm(b)
    if na < 1e-30 or nb < 1e-30:
        return 0.0
    return float(np.dot(a.flatten(), b.flatten()) / (na * nb))


def compute_compression_ratio(d: int, n_bits: int, group_size: int, jl_dim: int) -> float:
    """d * 16 / (16 + n_bits d + 32 ceil(d / group_size) + jl_dim) (utils.py:18-30)."""
    return d * 16 / (16 + n_bits * d + math.ceil(d / group_size) * 32 + jl_dim)


def attention_score_mse(scores_a: np.ndarray, scores_b: np.ndarray) -> float:
    return float(np.mean((scores_a - scores_b) ** 2))


def estimate_memory_bytes(batch: int, num_heads: int, seq_len: int, head_dim: int, n_bits: int, group_size: int,
                          jl_dim: int) -> int:
    """Bytes of the group format for batch x num_heads x seq_len vectors (utils.py:38-52)."""
    per_vector_bits = 16 + n_bits * head_dim + math.ceil(head_dim / group_size) * 32 + jl_dim
    return math.ceil(batch * num_heads * seq_len * per_vector_bits / 8)


def check_memory_warning(estimated_bytes: int) -> bool:
    """Whether the estimate exceeds 80 % of the available host memory (utils.py:55-58)."""
    import psutil
    return estimated_bytes > psutil.virtual_memory().available * 0.8
