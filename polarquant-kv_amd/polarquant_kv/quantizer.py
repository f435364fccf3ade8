"""PQ4 / PQ2 encoder entry points (device tensors only).

compress_pq is the codebook counterpart of the reference's compress_gpu
(src/polarquant_kv_cuda/compress_kernel.py:100-189) and of
turboquant_compress (csrc/flash_turboquant.cu:213-225): rotate, polar split,
nearest Lloyd-Max centroid per coordinate, pack into blocks, plus the optional
QJL key sketch. quantize_rotated is the bit-exact surface on fp32 rotated
input. Both call libpqkv_hip.so; there is no CPU path.
"""

from __future__ import annotations

import torch

from . import _lib
from .lloyd_max import padded_codebook_torch, stacked_codebooks_torch
from .types import PQCache, vector_bytes


def quantize_rotated(x_rot: torch.Tensor, codebook: torch.Tensor, n_bits: int = 4):
    """x_rot f32 [N, d] -> (blocks u8 [N, vector_bytes], radius f32 [N])."""
    _lib.require_device(x_rot, codebook)
    if x_rot.dtype != torch.float32 or x_rot.dim() != 2:
        raise ValueError("x_rot must be a 2-D float32 tensor")
    n, d = x_rot.shape
    x = x_rot.contiguous()
    cb = codebook.to(torch.float32).contiguous()
    blocks = torch.empty(n, vector_bytes(d, n_bits), dtype=torch.uint8, device=x.device)
    radius = torch.empty(n, dtype=torch.float32, device=x.device)
    _lib.check(_lib.lib().pqkv_quantize_rotated(x.data_ptr(), cb.data_ptr(), n_bits, blocks.data_ptr(),
                                                radius.data_ptr(), n, d, _lib.stream_of(x)))
    return blocks, radius


def allocate_cache(batch: int, num_heads: int, max_seq_len: int, head_dim: int, n_bits=4,
                   device="cuda", jl_dim: int = 0, codebooks=None) -> PQCache:
    """Empty cache of max_seq_len positions per (batch, head)."""
    mixed = not isinstance(n_bits, int)
    if mixed:
        if len(n_bits) != num_heads:
            raise ValueError("one width per head is required")
        per_batch = sum(max_seq_len * vector_bytes(head_dim, b) for b in n_bits)
        blocks = torch.zeros(batch, per_batch, dtype=torch.uint8, device=device)
        if codebooks is None:
            codebooks = stacked_codebooks_torch(head_dim, n_bits, device)
        n_bits = tuple(int(b) for b in n_bits)
    else:
        blocks = torch.zeros(batch, num_heads, max_seq_len, vector_bytes(head_dim, n_bits),
                             dtype=torch.uint8, device=device)
        if codebooks is None:
            codebooks = padded_codebook_torch(head_dim, n_bits, device)
    signs = None
    if jl_dim:
        signs = torch.zeros(batch, num_heads, max_seq_len, jl_dim // 8, dtype=torch.uint8, device=device)
    return PQCache(blocks=blocks, head_dim=head_dim, n_bits=n_bits, seq_len=0, max_seq_len=max_seq_len,
                   codebooks=codebooks, qjl_signs=signs, jl_dim=jl_dim)


def compress_pq(kv: torch.Tensor, rotation_matrix: torch.Tensor, n_bits=4, cache: PQCache | None = None,
                start: int | None = None, jl_rot: torch.Tensor | None = None) -> PQCache:
    """Encode kv [B, H, T, d] (fp16/fp32, device) into a PQ cache.

    With `cache`, positions start .. start+T-1 (default: cache.seq_len) are
    written in place and seq_len grows to cover them; otherwise a new cache of
    exactly T positions is returned. jl_rot = P R^T ([d, d] float32) adds the
    QJL sign sketch of each key's residual."""
    _lib.require_device(kv, rotation_matrix, jl_rot)
    if kv.dim() != 4:
        raise ValueError("kv must be [B, H, T, d]")
    B, H, T, d = kv.shape
    if cache is None:
        cache = allocate_cache(B, H, T, d, n_bits, kv.device, jl_dim=d if jl_rot is not None else 0)
        start = 0
    start = cache.seq_len if start is None else int(start)
    if cache.head_dim != d or cache.batch != B or cache.num_heads != H:
        raise ValueError("cache shape does not match kv")
    if start < 0 or start + T > cache.max_seq_len:
        raise ValueError(f"positions {start}..{start + T} exceed the cache capacity {cache.max_seq_len}")
    if jl_rot is not None and cache.qjl_signs is None:
        raise ValueError("cache was allocated without QJL signs")
    if T == 0:
        return cache
    x = kv.contiguous()
    R = rotation_matrix.to(torch.float32).contiguous()
    P = None if jl_rot is None else jl_rot.to(torch.float32).contiguous()
    stream = _lib.stream_of(x)
    lib = _lib.lib()
    es = x.element_size()
    if not cache.mixed:
        # (batch, head) pairs are the outer index: x rows T*d apart, cache
        # rows S_max vectors apart.
        vb = vector_bytes(d, cache.n_bits)
        qjl_ptr, qjl_stride = None, 0
        if P is not None:
            m8 = cache.qjl_signs.shape[-1]
            qjl_ptr = cache.qjl_signs.data_ptr() + start * m8
            qjl_stride = cache.max_seq_len * m8
        _lib.check(lib.pqkv_encode(x.data_ptr(), _lib.dtype_code(x.dtype), T * d, R.data_ptr(),
                                   cache.codebooks.data_ptr(), cache.n_bits,
                                   cache.blocks.data_ptr() + start * vb, cache.max_seq_len * vb, B * H, T, d,
                                   _lib.ptr(P), d if P is not None else 0, qjl_ptr, qjl_stride, stream))
    else:
        for h, bits in enumerate(cache.head_bits()):
            vb = vector_bytes(d, bits)
            base = cache.blocks.data_ptr() + cache.head_offset(h) + start * vb
            xq = x.data_ptr() + h * T * d * es
            qjl_ptr, qjl_stride = None, 0
            if P is not None:
                m8 = cache.qjl_signs.shape[-1]
                qjl_ptr = cache.qjl_signs.data_ptr() + ((h * cache.max_seq_len) + start) * m8
                qjl_stride = H * cache.max_seq_len * m8
            _lib.check(lib.pqkv_encode(xq, _lib.dtype_code(x.dtype), H * T * d, R.data_ptr(),
                                       cache.codebooks[h].data_ptr(), bits, base, cache.blocks.shape[1], B, T, d,
                                       _lib.ptr(P), d if P is not None else 0, qjl_ptr, qjl_stride, stream))
    cache.seq_len = max(cache.seq_len, start + T)
    return cache
