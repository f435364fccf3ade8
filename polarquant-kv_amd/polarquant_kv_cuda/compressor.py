"""High-level API (src/polarquant_kv_cuda/compressor.py:1-38)."""

from __future__ import annotations

from .attention_kernel import compressed_attention_gpu
from .compress_kernel import compress_gpu
from .decompress_kernel import decompress_gpu
from .types import CompressedKVCacheGPU


def compress(kv, rotation_matrix, n_bits=4, group_size=32, jl_matrix=None):
    return compress_gpu(kv, rotation_matrix, n_bits, group_size, jl_matrix)


def decompress(cache, rotation_matrix):
    return decompress_gpu(cache, rotation_matrix)


def compressed_attention(query, compressed_keys, compressed_values, rotation_matrix, jl_matrix=None,
                         enable_qjl=True, num_kv_heads=None):
    return compressed_attention_gpu(query, compressed_keys, compressed_values, rotation_matrix, jl_matrix,
                                    enable_qjl, num_kv_heads)


def get_memory_bytes(cache: CompressedKVCacheGPU) -> int:
    """Device bytes of the cache's tensors (compressor.py:28-38)."""
    total = 0
    for t in (cache.radius, cache.quantized_direction, cache.group_mins, cache.group_scales,
              cache.qjl_signs, cache.residual_norms):
        if t is not None:
            total += t.nelement() * t.element_size()
    return total
