"""KV cache manager on the group format (src/polarquant_kv_cuda/inference/kv_cache.py:14-134).

Same names, arguments and results as the reference's manager, which
compresses each append with compress_gpu and concatenates the whole cache
with torch.cat (kv_cache.py:93-116). Here the caches are allocated once for
max_seq_len positions at the first append and each append is encoded by the
HIP group encoder straight into its positions, so an append costs O(new
tokens). As in the reference, the manager writes no QJL signs
(kv_cache.py:112). memory_bytes counts the cached positions.
"""

from __future__ import annotations

import torch

from polarquant_kv.rotation import generate_rotation_matrix

from ..compress_kernel import compress_into, empty_cache
from ..types import CompressedKVCacheGPU
from .config import PolarQuantConfig


class KVCacheManager:
    """Compressed KV cache of one layer: prefill (several tokens) and decode
    (one token) appends."""

    def __init__(self, config: PolarQuantConfig, max_seq_len: int, batch: int, num_heads: int, head_dim: int,
                 device: str = "cuda", rotation_seed: int = 42):
        self.config = config
        self.max_seq_len = int(max_seq_len)
        self.batch = batch
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.device = device
        self.R = generate_rotation_matrix(head_dim, seed=rotation_seed, device=device)
        self._key_cache: torch.Tensor | None = None
        self._value_cache: torch.Tensor | None = None
        self._compressed_keys: CompressedKVCacheGPU | None = None
        self._compressed_values: CompressedKVCacheGPU | None = None
        self._seq_len = 0

    @property
    def seq_len(self) -> int:
        return self._seq_len

    def _position_bytes(self) -> int:
        c = self._compressed_keys
        per = 0
        for t in (c.radius, c.quantized_direction, c.group_mins, c.group_scales):
            per += t[0, 0, 0].nelement() * t.element_size()
        return per

    @property
    def memory_bytes(self) -> int:
        """Bytes of the cached positions (K + V)."""
        n = self.batch * self.num_heads * self._seq_len
        if not self.config.enable_compression:
            return 0 if self._key_cache is None else 2 * n * self.head_dim * 2
        if self._compressed_keys is None:
            return 0
        return 2 * n * self._position_bytes()

    @property
    def compression_ratio(self) -> float:
        if self._seq_len == 0:
            return 0.0
        original = self.batch * self.num_heads * self._seq_len * self.head_dim * 2 * 2
        compressed = self.memory_bytes
        return original / compressed if compressed > 0 else 0.0

    def append(self, key: torch.Tensor, value: torch.Tensor) -> None:
        """key / value [batch, num_heads, new_seq, head_dim] at positions
        seq_len .. seq_len + new_seq - 1."""
        B, H, T, d = key.shape
        if self._seq_len + T > self.max_seq_len:
            raise RuntimeError(f"KV cache full: {self._seq_len} + {T} > {self.max_seq_len}")
        if not self.config.enable_compression:
            if self._key_cache is None:
                shape = (B, H, self.max_seq_len, d)
                self._key_cache = torch.zeros(shape, dtype=key.dtype, device=key.device)
                self._value_cache = torch.zeros(shape, dtype=value.dtype, device=value.device)
            self._key_cache[:, :, self._seq_len:self._seq_len + T] = key
            self._value_cache[:, :, self._seq_len:self._seq_len + T] = value
        else:
            if self._compressed_keys is None:
                cfg = self.config
                self._compressed_keys = empty_cache(B, H, 0, d, cfg.n_bits, cfg.group_size, key.device,
                                                    max_seq_len=self.max_seq_len)
                self._compressed_values = empty_cache(B, H, 0, d, cfg.n_bits, cfg.group_size, key.device,
                                                      max_seq_len=self.max_seq_len)
            compress_into(self._compressed_keys, key, self.R, self._seq_len)
            compress_into(self._compressed_values, value, self.R, self._seq_len)
        self._seq_len += T

    def get_kv(self):
        """Compressed: the two CompressedKVCacheGPU (seq_len positions valid);
        uncompressed: views of the first seq_len positions."""
        if not self.config.enable_compression:
            if self._key_cache is None:
                return None, None
            return self._key_cache[:, :, :self._seq_len], self._value_cache[:, :, :self._seq_len]
        return self._compressed_keys, self._compressed_values

    def reset(self) -> None:
        """Forget the cached positions (the allocation is kept)."""
        self._seq_len = 0
        for c in (self._compressed_keys, self._compressed_values):
            if c is not None:
                c.seq_len = 0
