"""compress_gpu: the group (min / scale) format on the GPU
(src/polarquant_kv_cuda/compress_kernel.py:100-189), computed by
pqkv_group_gpu_compress and, for the QJL signs, pqkv_qjl_sketch.

Per vector (fp16 / bf16 / fp32 input, clamped to +-65000): y = x R^T, r = |y|,
u = y / max(r, 1e-30) (0 for a zero vector), zero-padded to whole groups;
per group lo = min, s = (max - lo) / (2^n_bits - 1) (1 for a flat group),
code = round_half_even(clamp((u - lo) / s, 0, 2^n_bits - 1)); stored radius,
lo and s in fp16, codes packed 4-bit / 2-bit or one byte per code. With a JL
matrix P [m, d]: signs of P e for the residual e = (y - y_hat) R (y_hat from
the unrounded lo, s and radius), and fp16 |e|.
"""

from __future__ import annotations

import math

import torch

from polarquant_kv import _lib

from .types import CompressedKVCacheGPU


def _validate_params(n_bits: int, group_size: int, d: int) -> None:
    """The reference's checks (compress_kernel.py:11-16)."""
    if not (2 <= n_bits <= 8):
        raise ValueError(f"n_bits must be in [2, 8], got {n_bits}")
    if group_size <= 0 or group_size > d:
        raise ValueError(f"invalid group_size {group_size} (d={d})")


def _packed_dim(d_padded: int, n_bits: int) -> int:
    if n_bits == 4:
        return d_padded // 2
    if n_bits == 2:
        return d_padded // 4
    return d_padded


def _bit_pack_quantized(quantized: torch.Tensor, n_bits: int) -> torch.Tensor:
    """[..., d_pad] uint8 codes -> packed rows (compress_kernel.py:19-63):
    4-bit (high << 4) | low, 2-bit v0 | v1<<2 | v2<<4 | v3<<6, other widths
    unchanged."""
    if n_bits not in (2, 4):
        return quantized
    q = quantized.to(torch.int32)
    if n_bits == 4:
        if q.shape[-1] % 2:
            raise ValueError("4-bit packing needs an even dimension")
        return (q[..., 0::2] | (q[..., 1::2] << 4)).to(torch.uint8)
    if q.shape[-1] % 4:
        raise ValueError("2-bit packing needs a dimension that is a multiple of 4")
    return (q[..., 0::4] | (q[..., 1::4] << 2) | (q[..., 2::4] << 4) | (q[..., 3::4] << 6)).to(torch.uint8)


def _bit_unpack_quantized(packed: torch.Tensor, n_bits: int, original_dim: int | None = None) -> torch.Tensor:
    """Inverse of _bit_pack_quantized (compress_kernel.py:66-97)."""
    if n_bits not in (2, 4):
        return packed
    p = packed.to(torch.int32)
    k = 2 if n_bits == 4 else 4
    mask = (1 << n_bits) - 1
    parts = [(p >> (n_bits * i)) & mask for i in range(k)]
    return torch.stack(parts, -1).reshape(*p.shape[:-1], p.shape[-1] * k).to(torch.uint8)


def _transposed(R: torch.Tensor) -> torch.Tensor:
    return R.t().contiguous()


def empty_cache(batch: int, heads: int, seq: int, d: int, n_bits: int, group_size: int, device, jl_dim: int = 0,
                max_seq_len: int | None = None) -> CompressedKVCacheGPU:
    """A group-format cache of max_seq_len (default seq) positions, seq_len = seq."""
    S = seq if max_seq_len is None else max_seq_len
    ng = math.ceil(d / group_size) if d > 0 else 0
    pd = _packed_dim(ng * group_size, n_bits)
    signs = norms = None
    if jl_dim:
        signs = torch.zeros(batch, heads, S, (jl_dim + 7) // 8, dtype=torch.uint8, device=device)
        norms = torch.zeros(batch, heads, S, dtype=torch.float16, device=device)
    return CompressedKVCacheGPU(
        radius=torch.zeros(batch, heads, S, dtype=torch.float16, device=device),
        quantized_direction=torch.zeros(batch, heads, S, pd, dtype=torch.uint8, device=device),
        group_mins=torch.zeros(batch, heads, S, ng, dtype=torch.float16, device=device),
        group_scales=torch.zeros(batch, heads, S, ng, dtype=torch.float16, device=device),
        qjl_signs=signs, residual_norms=norms, n_bits=n_bits, group_size=group_size, original_dim=d,
        seq_len=seq, max_seq_len=S)


def _compress_rows(x: torch.Tensor, R: torch.Tensor, n_bits: int, group_size: int, jl_matrix, out: dict) -> None:
    """x [n, d] device -> the fields in `out` (contiguous [n, ...] tensors)."""
    n, d = x.shape
    lib = _lib.lib()
    stream = _lib.stream_of(x)
    dt = x.dtype
    if dt not in (torch.float16, torch.float32, torch.bfloat16):
        x = x.float()
    code = {torch.float16: _lib.F16, torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}[x.dtype]
    Rf = R.to(device=x.device, dtype=torch.float32).contiguous()
    resid = torch.empty(n, d, dtype=torch.float32, device=x.device) if jl_matrix is not None else None
    _lib.check(lib.pqkv_group_gpu_compress(x.data_ptr(), code, Rf.data_ptr(), _transposed(Rf).data_ptr(), n, d,
                                           n_bits, group_size, out["radius"].data_ptr(), out["codes"].data_ptr(),
                                           out["mins"].data_ptr(), out["scales"].data_ptr(), _lib.F16,
                                           _lib.ptr(resid), stream))
    if jl_matrix is not None:
        P = torch.as_tensor(jl_matrix).to(device=x.device, dtype=torch.float64)
        m = P.shape[0]
        Pt = P.t().contiguous()
        _lib.check(lib.pqkv_qjl_sketch(resid.data_ptr(), _lib.F32, None, Pt.data_ptr(), n, d, m,
                                       out["signs"].data_ptr(), out["norms"].data_ptr(), _lib.F16, stream))


def compress_gpu(kv: torch.Tensor, rotation_matrix: torch.Tensor, n_bits: int = 4, group_size: int = 32,
                 jl_matrix: torch.Tensor | None = None) -> CompressedKVCacheGPU:
    """kv [batch, heads, seq, d] on the GPU -> CompressedKVCacheGPU with
    seq_len = max_seq_len = seq (compress_kernel.py:100-189). An empty kv
    gives an empty cache of the input's shape."""
    if kv.numel() == 0:
        batch = kv.shape[0] if kv.dim() >= 1 else 0
        heads = kv.shape[1] if kv.dim() >= 2 else 0
        seq = kv.shape[2] if kv.dim() >= 3 else 0
        d = kv.shape[3] if kv.dim() >= 4 else 0
        c = empty_cache(batch, heads, seq, d, n_bits, group_size, kv.device)
        return c
    if kv.dim() != 4:
        raise ValueError("kv must be [batch, num_heads, seq_len, head_dim]")
    _lib.require_device(kv)
    B, H, S, d = kv.shape
    _validate_params(n_bits, group_size, d)
    m = 0 if jl_matrix is None else int(jl_matrix.shape[0])
    cache = empty_cache(B, H, S, d, n_bits, group_size, kv.device, jl_dim=m)
    out = {"radius": cache.radius, "codes": cache.quantized_direction, "mins": cache.group_mins,
           "scales": cache.group_scales, "signs": cache.qjl_signs, "norms": cache.residual_norms}
    _compress_rows(kv.reshape(-1, d).contiguous(), rotation_matrix, n_bits, group_size, jl_matrix, out)
    return cache


def compress_into(cache: CompressedKVCacheGPU, kv: torch.Tensor, rotation_matrix: torch.Tensor, start: int,
                  jl_matrix: torch.Tensor | None = None) -> CompressedKVCacheGPU:
    """Encode kv [B, H, T, d] into positions start .. start + T - 1 of a
    preallocated cache (seq_len grows to cover them)."""
    B, H, T, d = kv.shape
    if start < 0 or start + T > cache.max_seq_len:
        raise ValueError(f"positions {start}..{start + T} exceed the cache capacity {cache.max_seq_len}")
    if T == 0:
        return cache
    if jl_matrix is not None and cache.qjl_signs is None:
        raise ValueError("cache was allocated without QJL signs")
    tmp = compress_gpu(kv, rotation_matrix, cache.n_bits, cache.group_size, jl_matrix)
    sl = slice(start, start + T)
    cache.radius[:, :, sl] = tmp.radius
    cache.quantized_direction[:, :, sl] = tmp.quantized_direction
    cache.group_mins[:, :, sl] = tmp.group_mins
    cache.group_scales[:, :, sl] = tmp.group_scales
    if jl_matrix is not None:
        cache.qjl_signs[:, :, sl] = tmp.qjl_signs
        cache.residual_norms[:, :, sl] = tmp.residual_norms
    cache.seq_len = max(cache.seq_len, start + T)
    return cache
