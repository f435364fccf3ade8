"""PQ4 / PQ2 encoder and decoder entry points (device tensors only).

compress_pq is the codebook counterpart of the reference's compress_gpu
(src/polarquant_kv_cuda/compress_kernel.py:100-189) and of
turboquant_compress (csrc/flash_turboquant.cu:213-225): rotate, polar split,
nearest Lloyd-Max centroid per coordinate, pack into blocks, plus the optional
QJL key sketch. compress_gpu / decompress_gpu keep the reference's names and
arguments for that format; dequantize is the general decoder. quantize_rotated
is the bit-exact surface on fp32 rotated input. All call libpqkv_hip.so;
there is no CPU path.
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


def _validate_params(n_bits: int, group_size: int, d: int) -> None:
    """The reference's argument checks (python/polarquant_kv/quantizer.py:15-22,
    src/polarquant_kv_cuda/compress_kernel.py:13-20), same messages' meaning."""
    if not (2 <= n_bits <= 8):
        raise ValueError(f"n_bits must be in [2, 8], got {n_bits}")
    if group_size <= 0:
        raise ValueError(f"group_size must be positive, got {group_size}")
    if group_size > d:
        raise ValueError(f"group_size ({group_size}) cannot exceed the vector dimension d ({d})")


def compress_gpu(kv: torch.Tensor, rotation_matrix: torch.Tensor, n_bits: int = 4, group_size: int = 32,
                 jl_matrix=None) -> PQCache:
    """The reference's compress_gpu entry point
    (src/polarquant_kv_cuda/compress_kernel.py:100-189) for the codebook
    (PQ4 / PQ2) format: kv [B, H, S, d] -> a PQCache of exactly S positions.
    The codebook format's block is 32 coordinates; group_size is checked like
    the reference's and otherwise has no effect. jl_matrix (P, [d, d]) adds
    the QJL signs of each vector's residual (compress_kernel.py:166-175).
    Empty input gives an empty cache with the input's shape."""
    if kv.dim() != 4:
        raise ValueError("kv must be [batch, heads, seq, head_dim]")
    B, H, S, d = kv.shape
    _validate_params(n_bits, group_size, max(d, 1))
    if n_bits not in (2, 4):
        raise ValueError(f"the codebook format stores 2- or 4-bit codes, got n_bits={n_bits}")
    jl_rot = None
    if jl_matrix is not None:
        from .qjl import rotated_jl_matrix
        jl_rot = rotated_jl_matrix(jl_matrix, rotation_matrix, kv.device)
    if kv.numel() == 0:
        return allocate_cache(B, H, S, d, n_bits, kv.device, jl_dim=d if jl_rot is not None else 0)
    return compress_pq(kv, rotation_matrix, n_bits, jl_rot=jl_rot)


def dequantize(cache: PQCache, rotation_matrix: torch.Tensor | None, out_dtype=torch.float16,
               positions: int | None = None) -> torch.Tensor:
    """Reconstruction r16 c[code] of the first `positions` (default seq_len)
    positions of every (batch, head), rotated back with R (pqkv_dequantize):
    [B, H, positions, d] of out_dtype. rotation_matrix None leaves the
    rotated-space reconstruction (R = I, exact)."""
    S = cache.seq_len if positions is None else int(positions)
    B, H, d = cache.batch, cache.num_heads, cache.head_dim
    dev = cache.blocks.device
    R = (torch.eye(d, device=dev) if rotation_matrix is None else rotation_matrix).to(torch.float32).contiguous()
    _lib.require_device(cache.blocks, R)
    out = torch.empty(B, H, S, d, dtype=out_dtype, device=dev)
    if S == 0:
        return out
    lib = _lib.lib()
    stream = _lib.stream_of(out)
    for b in range(B):
        for h, bits in enumerate(cache.head_bits()):
            vb = vector_bytes(d, bits)
            if cache.mixed:
                src = cache.blocks[b].data_ptr() + cache.head_offset(h)
                cb = cache.codebooks[h] if cache.codebooks.dim() == 2 else cache.codebooks
            else:
                if h > 0:
                    continue
                # uniform widths: every head of the batch row in one call when
                # the rows are contiguous (S == max_seq_len), else per head
                cb = cache.codebooks
                if S == cache.max_seq_len:
                    _lib.check(lib.pqkv_dequantize(cache.blocks[b].data_ptr(), cb.data_ptr(), bits, R.data_ptr(),
                                                   out[b].data_ptr(), _lib.dtype_code(out_dtype), H * S, d, stream))
                    continue
                for hh in range(H):
                    _lib.check(lib.pqkv_dequantize(cache.blocks[b, hh].data_ptr(), cb.data_ptr(), bits,
                                                   R.data_ptr(), out[b, hh].data_ptr(), _lib.dtype_code(out_dtype),
                                                   S, d, stream))
                continue
            _lib.check(lib.pqkv_dequantize(src, cb.data_ptr(), bits, R.data_ptr(), out[b, h].data_ptr(),
                                           _lib.dtype_code(out_dtype), S, d, stream))
    return out


def decompress_gpu(cache: PQCache, rotation_matrix: torch.Tensor) -> torch.Tensor:
    """The reference's decompress_gpu (src/polarquant_kv_cuda/decompress_kernel.py:10-55)
    for the codebook format: fp16 [B, H, seq_len, d] in the original space,
    saturated at +-65504; an empty cache gives an empty tensor."""
    return dequantize(cache, rotation_matrix, torch.float16)
