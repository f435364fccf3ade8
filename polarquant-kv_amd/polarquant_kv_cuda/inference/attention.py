"""Compressed multi-head attention layer (src/polarquant_kv_cuda/inference/attention.py:12-92).

The reference's semantics: queries, keys and values in fp16; with a cache
manager the new keys and values are appended and every query attends to the
whole cache (no causal mask, as the reference's calls); the compressed path
runs compressed_attention_gpu on the group-format caches (here the fused
kernel), the uncompressed paths torch's SDPA.
"""

from __future__ import annotations

import torch

from ..attention_kernel import compressed_attention_gpu
from .config import PolarQuantConfig
from .kv_cache import KVCacheManager


class CompressedMultiHeadAttention(torch.nn.Module):
    def __init__(self, config: PolarQuantConfig, embed_dim: int, num_heads: int, num_kv_heads: int | None = None):
        super().__init__()
        self.config = config
        self.embed_dim = embed_dim
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads or num_heads
        self.head_dim = embed_dim // num_heads
        self.q_proj = torch.nn.Linear(embed_dim, num_heads * self.head_dim, bias=False)
        self.k_proj = torch.nn.Linear(embed_dim, self.num_kv_heads * self.head_dim, bias=False)
        self.v_proj = torch.nn.Linear(embed_dim, self.num_kv_heads * self.head_dim, bias=False)
        self.o_proj = torch.nn.Linear(num_heads * self.head_dim, embed_dim, bias=False)

    def _heads(self, t: torch.Tensor, n: int) -> torch.Tensor:
        B, T, _ = t.shape
        return t.reshape(B, T, n, self.head_dim).transpose(1, 2).half()

    def forward(self, x: torch.Tensor, cache_manager: KVCacheManager | None = None) -> torch.Tensor:
        """x [batch, seq_len, embed_dim] -> [batch, seq_len, embed_dim]."""
        B, T, _ = x.shape
        q = self._heads(self.q_proj(x), self.num_heads)
        k = self._heads(self.k_proj(x), self.num_kv_heads)
        v = self._heads(self.v_proj(x), self.num_kv_heads)
        if cache_manager is not None:
            cache_manager.append(k, v)
            out = self._attend_with_cache(q, cache_manager)
        else:
            out = self._attend_standard(q, k, v)
        return self.o_proj(out.transpose(1, 2).reshape(B, T, -1).float())

    def _attend_standard(self, q, k, v):
        return self._sdpa(q, k, v)

    def _sdpa(self, q, k, v):
        if k.shape[1] < q.shape[1]:
            rep = q.shape[1] // k.shape[1]
            k = k.repeat_interleave(rep, dim=1)
            v = v.repeat_interleave(rep, dim=1)
        return torch.nn.functional.scaled_dot_product_attention(q.float(), k.float(), v.float()).half()

    def _attend_with_cache(self, q, cache_manager: KVCacheManager):
        ck, cv = cache_manager.get_kv()
        if not cache_manager.config.enable_compression:
            return self._sdpa(q, ck, cv)
        return compressed_attention_gpu(q, ck, cv, cache_manager.R)
