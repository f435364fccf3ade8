"""Small test transformer (src/polarquant_kv_cuda/inference/transformer.py:11-66):
pre-norm layers of the compressed attention and a GELU MLP, with one cache
manager per layer (rotation seeds 42 + layer)."""

from __future__ import annotations

import torch

from .attention import CompressedMultiHeadAttention
from .config import PolarQuantConfig
from .kv_cache import KVCacheManager


class SimpleTransformerLayer(torch.nn.Module):
    def __init__(self, config: PolarQuantConfig, embed_dim: int, num_heads: int, num_kv_heads: int | None = None,
                 ffn_dim: int | None = None):
        super().__init__()
        hidden = ffn_dim or 4 * embed_dim
        self.attn = CompressedMultiHeadAttention(config, embed_dim, num_heads, num_kv_heads)
        self.norm1 = torch.nn.LayerNorm(embed_dim)
        self.norm2 = torch.nn.LayerNorm(embed_dim)
        self.ffn = torch.nn.Sequential(torch.nn.Linear(embed_dim, hidden, bias=False), torch.nn.GELU(),
                                       torch.nn.Linear(hidden, embed_dim, bias=False))

    def forward(self, x: torch.Tensor, cache_manager: KVCacheManager | None = None) -> torch.Tensor:
        x = x + self.attn(self.norm1(x.float()), cache_manager)
        return x + self.ffn(self.norm2(x.float()))


class SimpleTransformer(torch.nn.Module):
    def __init__(self, config: PolarQuantConfig, num_layers: int, embed_dim: int, num_heads: int,
                 num_kv_heads: int | None = None, vocab_size: int = 1000):
        super().__init__()
        self.config = config
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads or num_heads
        self.head_dim = embed_dim // num_heads
        self.embed = torch.nn.Embedding(vocab_size, embed_dim)
        self.layers = torch.nn.ModuleList(SimpleTransformerLayer(config, embed_dim, num_heads, num_kv_heads)
                                          for _ in range(num_layers))
        self.head = torch.nn.Linear(embed_dim, vocab_size, bias=False)

    def forward(self, input_ids: torch.Tensor, cache_managers: list | None = None) -> torch.Tensor:
        x = self.embed(input_ids).float()
        for i, layer in enumerate(self.layers):
            x = layer(x, cache_managers[i] if cache_managers else None)
        return self.head(x.float())

    def create_cache_managers(self, max_seq_len: int, batch: int, device: str = "cuda") -> list:
        return [KVCacheManager(self.config, max_seq_len, batch, self.num_kv_heads, self.head_dim, device,
                               rotation_seed=42 + i) for i in range(len(self.layers))]
