"""Containers of the GPU group format (src/polarquant_kv_cuda/types.py:7-21)."""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass
class CompressedKVCacheGPU:
    """A group-format KV cache on the GPU, the reference's fields and dtypes.
    Tensors are [batch, num_heads, max_seq_len, ...]; positions 0 ..
    seq_len - 1 are valid (the reference's compress_gpu sets seq_len ==
    max_seq_len; a preallocated cache grows seq_len in place)."""

    radius: torch.Tensor                   # [B, H, S_max] fp16
    quantized_direction: torch.Tensor      # [B, H, S_max, packed] uint8 (4-bit: d_pad/2, 2-bit: d_pad/4, else d_pad)
    group_mins: torch.Tensor               # [B, H, S_max, num_groups] fp16
    group_scales: torch.Tensor             # [B, H, S_max, num_groups] fp16
    qjl_signs: torch.Tensor | None         # [B, H, S_max, ceil(jl_dim / 8)] uint8
    residual_norms: torch.Tensor | None    # [B, H, S_max] fp16
    n_bits: int
    group_size: int
    original_dim: int
    seq_len: int
    max_seq_len: int
