"""decompress_gpu (src/polarquant_kv_cuda/decompress_kernel.py:10-51) on the
GPU: x^ = clamp(((code s + lo) r) R, +-65504) in fp16, by
pqkv_group_gpu_decompress."""

from __future__ import annotations

import torch

from polarquant_kv import _lib

from .types import CompressedKVCacheGPU


def decompress_gpu(cache: CompressedKVCacheGPU, rotation_matrix: torch.Tensor) -> torch.Tensor:
    """[batch, heads, seq_len, original_dim] fp16; a cache of seq_len 0 gives
    an empty tensor."""
    B, H = cache.radius.shape[0], cache.radius.shape[1]
    d, S = cache.original_dim, cache.seq_len
    out = torch.empty(B, H, S, d, dtype=torch.float16, device=cache.radius.device)
    if S == 0 or B * H == 0:
        return out
    full = S == cache.radius.shape[2]

    def rows(t):
        t = t if full else t[:, :, :S]
        return t.contiguous()

    r, c, lo, sc = rows(cache.radius), rows(cache.quantized_direction), rows(cache.group_mins), rows(
        cache.group_scales)
    R = rotation_matrix.to(device=out.device, dtype=torch.float32).contiguous()
    _lib.check(_lib.lib().pqkv_group_gpu_decompress(r.data_ptr(), c.data_ptr(), lo.data_ptr(), sc.data_ptr(),
                                                    _lib.F16, R.data_ptr(), B * H * S, d, cache.n_bits,
                                                    cache.group_size, out.data_ptr(), _lib.F16,
                                                    _lib.stream_of(out)))
    return out
