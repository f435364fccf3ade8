"""Inference-side cache and attention layer on the compressed format.

Mirrors src/polarquant_kv_cuda/inference/{config,kv_cache,attention}.py of
the reference with the same names and arguments:

  PolarQuantConfig             n_bits, group_size, jl_dim, enable_qjl,
                               enable_compression (config.py)
  KVCacheManager               append / get_kv / reset / seq_len /
                               memory_bytes / compression_ratio (kv_cache.py:14-134)
  CompressedMultiHeadAttention q/k/v/o projections, forward(x, cache_manager)
                               (attention.py:12-95)

Differences, all on purpose:
  - the compressed caches are paged (PagedPQCache): they grow by pages of
    page_tokens positions as the sequence grows, and append encodes the new
    positions straight into their pages through the page table
    (pqkv_encode_paged), never copying what is cached (the reference
    concatenates the whole cache with torch.cat on every append,
    kv_cache.py:96-116), so a decode step costs O(new tokens), not O(S), and
    memory follows the sequence, not max_seq_len (a limit only); attention
    runs the paged decode / chunked-prefill kernels;
  - the layout is block_pq4 / block_pq2 with Lloyd-Max centroids (the
    reference manager stores its per-group min/scale format);
  - with enable_qjl the keys carry the QJL sign sketch and attention adds
    the correction (the reference manager never writes signs, kv_cache.py:112);
  - CompressedMultiHeadAttention applies the causal rule to a multi-token
    chunk on every path (query i of a chunk at positions p0.. sees positions
    <= p0 + i): the compressed cache, the uncompressed cache and no cache.
    The reference calls non-causal SDPA / compressed attention on all three
    (inference/attention.py:63-92), so a chunk's queries see its later
    tokens; causal=False reproduces that.
All GPU work goes through libpqkv_hip.so.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import attention, quantizer
from .types import PagedPQCache


@dataclass
class PolarQuantConfig:
    n_bits: int = 4
    group_size: int = 32
    jl_dim: int = 64
    enable_qjl: bool = False
    enable_compression: bool = True


class KVCacheManager:
    """Compressed KV cache of one attention layer: up to max_seq_len
    positions per (batch, head), kept in pages of page_tokens positions
    (a power of two, >= 64), filled by prefill (several tokens) and decode
    (one token) appends."""

    def __init__(self, config: PolarQuantConfig, max_seq_len: int, batch: int, num_heads: int, head_dim: int,
                 device: str = "cuda", rotation_seed: int = 42, page_tokens: int = 256):
        from .rotation import generate_rotation_matrix
        if config.enable_compression:
            quantizer._validate_params(config.n_bits, config.group_size, head_dim)
            if config.n_bits not in (2, 4):
                raise ValueError(f"the codebook format stores 2- or 4-bit codes, got n_bits={config.n_bits}")
        self.config = config
        self.page_tokens = int(page_tokens)
        self.max_seq_len = int(max_seq_len)
        self.batch = batch
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.device = device
        self.R = generate_rotation_matrix(head_dim, seed=rotation_seed, device=device)
        self.jl_rot = None
        if config.enable_compression and config.enable_qjl:
            if config.jl_dim != head_dim:
                raise ValueError(f"the QJL sketch here has m = head_dim projections (jl_dim={config.jl_dim}, "
                                 f"head_dim={head_dim})")
            from .qjl import generate_jl_matrix, rotated_jl_matrix
            self.jl_matrix = generate_jl_matrix(config.jl_dim, head_dim, seed=rotation_seed + 1)
            self.jl_rot = rotated_jl_matrix(self.jl_matrix, self.R.cpu().numpy(), device)
        self._keys: PagedPQCache | None = None
        self._values: PagedPQCache | None = None
        self._key_cache: torch.Tensor | None = None
        self._value_cache: torch.Tensor | None = None
        self._seq_len = 0

    # ---- allocation ----
    def _allocate(self):
        if self.config.enable_compression:
            B, H, d, bits = self.batch, self.num_heads, self.head_dim, self.config.n_bits
            self._keys = quantizer.allocate_paged_cache(B, H, d, bits, self.device, page_tokens=self.page_tokens,
                                                        jl_dim=d if self.jl_rot is not None else 0)
            self._values = quantizer.allocate_paged_cache(B, H, d, bits, self.device, page_tokens=self.page_tokens)
        else:
            shape = (self.batch, self.num_heads, self.max_seq_len, self.head_dim)
            self._key_cache = torch.zeros(shape, dtype=torch.float16, device=self.device)
            self._value_cache = torch.zeros(shape, dtype=torch.float16, device=self.device)

    @property
    def seq_len(self) -> int:
        return self._seq_len

    @property
    def memory_bytes(self) -> int:
        """Bytes of the cached positions (K + V, and the QJL signs)."""
        if self._seq_len == 0:
            return 0
        n = self.batch * self.num_heads * self._seq_len
        if not self.config.enable_compression:
            return 2 * n * self.head_dim * 2
        from .types import vector_bytes
        per = 2 * vector_bytes(self.head_dim, self.config.n_bits)
        if self.jl_rot is not None:
            per += self.head_dim // 8
        return n * per

    @property
    def allocated_bytes(self) -> int:
        """Device bytes held: the pages allocated so far (and their tables);
        uncompressed, the max_seq_len-position arrays."""
        if self.config.enable_compression:
            return 0 if self._keys is None else self._keys.memory_bytes() + self._values.memory_bytes()
        return 0 if self._key_cache is None else 2 * self._key_cache.numel() * 2

    @property
    def compression_ratio(self) -> float:
        if self._seq_len == 0:
            return 0.0
        original = self.batch * self.num_heads * self._seq_len * self.head_dim * 2 * 2   # K + V, fp16
        return original / self.memory_bytes

    # ---- writes ----
    def append(self, key: torch.Tensor, value: torch.Tensor) -> None:
        """key / value [batch, num_heads, new_seq, head_dim] (fp16 or fp32) at
        positions seq_len .. seq_len + new_seq - 1, encoded into their pages
        (pages are added as the positions need them)."""
        if key.shape != value.shape or key.dim() != 4:
            raise ValueError("key and value must both be [batch, num_heads, new_seq, head_dim]")
        B, H, T, d = key.shape
        if (B, H, d) != (self.batch, self.num_heads, self.head_dim):
            raise ValueError(f"shape {tuple(key.shape)} does not match the cache "
                             f"({self.batch}, {self.num_heads}, *, {self.head_dim})")
        if self._seq_len + T > self.max_seq_len:
            raise RuntimeError(f"KV cache full: {self._seq_len} + {T} > {self.max_seq_len}")
        if self._keys is None and self._key_cache is None:
            self._allocate()
        if self.config.enable_compression:
            quantizer.compress_pq(key, self.R, cache=self._keys, start=self._seq_len, jl_rot=self.jl_rot)
            quantizer.compress_pq(value, self.R, cache=self._values, start=self._seq_len)
        else:
            self._key_cache[:, :, self._seq_len:self._seq_len + T] = key.to(torch.float16)
            self._value_cache[:, :, self._seq_len:self._seq_len + T] = value.to(torch.float16)
        self._seq_len += T

    def get_kv(self):
        """Compressed: the two PagedPQCache objects (seq_len positions valid);
        uncompressed: views of the first seq_len positions."""
        if not self.config.enable_compression:
            if self._key_cache is None:
                return None, None
            return self._key_cache[:, :, :self._seq_len], self._value_cache[:, :, :self._seq_len]
        return self._keys, self._values

    def reset(self) -> None:
        """Forget the cached positions (the pages are kept for reuse)."""
        self._seq_len = 0
        for c in (self._keys, self._values):
            if c is not None:
                c.seq_len = 0

    # ---- reads ----
    def attend(self, query: torch.Tensor, causal: bool = True) -> torch.Tensor:
        """query [batch, q_heads, Sq, head_dim] for the last Sq cached
        positions -> [batch, q_heads, Sq, head_dim] fp16: compressed
        attention (decode for Sq = 1, causal prefill otherwise) with the QJL
        term when the manager keeps signs."""
        if self._seq_len == 0:
            return torch.zeros_like(query, dtype=torch.float16)
        if not self.config.enable_compression:
            k, v = self.get_kv()
            rep = query.shape[1] // k.shape[1]
            k = k.float().repeat_interleave(rep, 1)
            v = v.float().repeat_interleave(rep, 1)
            Sq, S = query.shape[2], k.shape[2]
            s = torch.matmul(query.float(), k.transpose(-1, -2).contiguous()) / math.sqrt(self.head_dim)
            if causal and Sq > 1:
                pos = torch.arange(S, device=query.device)
                qpos = torch.arange(S - Sq, S, device=query.device)
                s = s.masked_fill(pos[None, :] > qpos[:, None], float("-inf"))
            return torch.matmul(torch.softmax(s, -1), v).half()
        Sq = query.shape[2]
        jl = self.jl_matrix if self.jl_rot is not None else None
        return attention.compressed_attention_gpu(query, self._keys, self._values, self.R, jl_matrix=jl,
                                                  causal=causal, q_start=self._seq_len - Sq)


class CompressedMultiHeadAttention(torch.nn.Module):
    """Multi-head (GQA) attention whose KV cache is the compressed one
    (src/polarquant_kv_cuda/inference/attention.py:12-95)."""

    def __init__(self, config: PolarQuantConfig, embed_dim: int, num_heads: int, num_kv_heads: int | None = None,
                 causal: bool = True):
        super().__init__()
        self.config = config
        self.causal = causal
        self.embed_dim = embed_dim
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads or num_heads
        self.head_dim = embed_dim // num_heads
        self.q_proj = torch.nn.Linear(embed_dim, num_heads * self.head_dim, bias=False)
        self.k_proj = torch.nn.Linear(embed_dim, self.num_kv_heads * self.head_dim, bias=False)
        self.v_proj = torch.nn.Linear(embed_dim, self.num_kv_heads * self.head_dim, bias=False)
        self.o_proj = torch.nn.Linear(num_heads * self.head_dim, embed_dim, bias=False)

    def forward(self, x: torch.Tensor, cache_manager: KVCacheManager | None = None) -> torch.Tensor:
        """x [batch, seq_len, embed_dim] -> [batch, seq_len, embed_dim]. With a
        cache manager the new keys and values are appended and the queries
        attend to everything cached (causally unless causal=False)."""
        B, T, _ = x.shape
        q = self.q_proj(x).reshape(B, T, self.num_heads, self.head_dim).transpose(1, 2).half()
        k = self.k_proj(x).reshape(B, T, self.num_kv_heads, self.head_dim).transpose(1, 2).half()
        v = self.v_proj(x).reshape(B, T, self.num_kv_heads, self.head_dim).transpose(1, 2).half()
        if cache_manager is not None:
            cache_manager.append(k.contiguous(), v.contiguous())
            out = cache_manager.attend(q.contiguous(), causal=self.causal)
        else:
            rep = self.num_heads // self.num_kv_heads
            kk = k.float().repeat_interleave(rep, 1)
            vv = v.float().repeat_interleave(rep, 1)
            s = torch.matmul(q.float(), kk.transpose(-1, -2).contiguous()) / math.sqrt(self.head_dim)
            if self.causal:
                mask = torch.ones(T, T, dtype=torch.bool, device=x.device).triu(1)
                s = s.masked_fill(mask, float("-inf"))
            out = torch.matmul(torch.softmax(s, -1), vv).half()
        out = out.transpose(1, 2).reshape(B, T, -1)
        return self.o_proj(out.to(self.o_proj.weight.dtype))
