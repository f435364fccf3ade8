"""compressed_attention_gpu (src/polarquant_kv_cuda/attention_kernel.py:11-113).

On group-format caches (CompressedKVCacheGPU) the attention runs straight on
the packed codes by pqkv_group_attn: query rotation, a split-K kernel that
forms s_t = scale r_t sum_g (s_tg q_rot.c_tg + lo_tg sum_{j in g} q_rot_j)
(+ the QJL term, none for a zero residual) and o_rot = sum_t w_t r_t (c_t s_t
+ lo_t), then the split merge with the inverse rotation. The reference
decompresses both caches to fp16 and runs dense matmuls instead; the
results agree to that fp16 rounding. Every query token attends to every
cached position, as there. On PQCache caches (the codebook format) this is
polarquant_kv.attention.compressed_attention_gpu.
"""

from __future__ import annotations

import torch

from polarquant_kv import _lib
from polarquant_kv.types import PQCache

from .types import CompressedKVCacheGPU


def group_attention(query: torch.Tensor, keys: CompressedKVCacheGPU, values: CompressedKVCacheGPU,
                    rotation_matrix: torch.Tensor, jl_matrix=None, enable_qjl: bool = True,
                    scale: float | None = None, out_dtype=None) -> torch.Tensor:
    """query [B, Hq, Sq, d] (or [B, Hq, d]) against two group-format caches
    of the same shape -> the query's shape in out_dtype (default the
    query's dtype)."""
    squeeze = query.dim() == 3
    q = query[:, :, None] if squeeze else query
    if q.dim() != 4:
        raise ValueError("query must be [batch, q_heads, seq_q, head_dim]")
    B, Hq, Sq, d = q.shape
    out_dtype = query.dtype if out_dtype is None else out_dtype
    if out_dtype not in (torch.float16, torch.float32):
        out_dtype = torch.float32
    Hkv, S = keys.radius.shape[1], keys.seq_len
    if keys.original_dim != d or values.original_dim != d:
        raise ValueError(f"head_dim {d} does not match the caches ({keys.original_dim})")
    if keys.radius.shape[:2] != (B, Hkv) or values.radius.shape[:2] != (B, Hkv) or values.seq_len != S:
        raise ValueError("key and value caches must have the same batch, heads and length")
    if Hq % Hkv:
        raise ValueError(f"query heads {Hq} are not a multiple of kv heads {Hkv}")
    if (keys.n_bits, keys.group_size) != (values.n_bits, values.group_size):
        raise ValueError("key and value caches must share n_bits and group_size")
    _lib.require_device(q, keys.radius, values.radius)
    out = torch.empty(B, Hq, Sq, d, dtype=out_dtype, device=q.device)
    if S == 0:
        out.zero_()
        return out[:, :, 0] if squeeze else out
    qc = q if q.dtype in (torch.float16, torch.float32, torch.bfloat16) else q.float()
    qc = qc.contiguous()
    qcode = {torch.float16: _lib.F16, torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}[qc.dtype]
    R = rotation_matrix.to(device=q.device, dtype=torch.float32).contiguous()
    use_qjl = enable_qjl and jl_matrix is not None and keys.qjl_signs is not None
    P = torch.as_tensor(jl_matrix).to(device=q.device, dtype=torch.float32).contiguous() if use_qjl else None
    m = int(P.shape[0]) if use_qjl else 0
    if use_qjl and keys.qjl_signs.shape[-1] * 8 < m:
        raise ValueError("the cache's sign sketch is shorter than the JL matrix")
    scale = float(d) ** -0.5 if scale is None else float(scale)
    rows = Hq * Sq
    lib = _lib.lib()
    ws = torch.empty(lib.pqkv_group_attn_workspace_bytes(B, rows, Hkv, S, d, keys.group_size, m),
                     dtype=torch.uint8, device=q.device)
    pdt = _lib.dtype_code(keys.radius.dtype)
    for f in (keys.group_mins, keys.group_scales, values.radius, values.group_mins, values.group_scales):
        if f.dtype != keys.radius.dtype:
            raise ValueError("the caches' radius, minima and scales must share one dtype")
    for t in (keys.radius, keys.quantized_direction, keys.group_mins, keys.group_scales, values.radius,
              values.quantized_direction, values.group_mins, values.group_scales):
        if not t.is_contiguous():
            raise ValueError("cache fields must be contiguous [B, H, S_max, ...] tensors")
    signs = keys.qjl_signs.contiguous() if use_qjl else None
    norms = keys.residual_norms.contiguous() if use_qjl and keys.residual_norms is not None else None
    if norms is not None and norms.dtype != keys.radius.dtype:
        norms = norms.to(keys.radius.dtype)
    _lib.check(lib.pqkv_group_attn(qc.data_ptr(), qcode, R.data_ptr(), _lib.ptr(P), m,
                                   keys.quantized_direction.data_ptr(), keys.radius.data_ptr(),
                                   keys.group_mins.data_ptr(), keys.group_scales.data_ptr(),
                                   values.quantized_direction.data_ptr(), values.radius.data_ptr(),
                                   values.group_mins.data_ptr(), values.group_scales.data_ptr(),
                                   _lib.ptr(signs), _lib.ptr(norms), keys.n_bits, pdt, B, rows, Hkv, S,
                                   keys.radius.shape[2], d, keys.group_size, scale, out.data_ptr(),
                                   _lib.dtype_code(out_dtype), ws.data_ptr(), ws.numel(), _lib.stream_of(q)))
    return out[:, :, 0] if squeeze else out


def compressed_attention_gpu(query: torch.Tensor, compressed_keys, compressed_values, rotation_matrix: torch.Tensor,
                             jl_matrix: torch.Tensor | None = None, enable_qjl: bool = True,
                             num_kv_heads: int | None = None) -> torch.Tensor:
    """query [B, Hq, Sq, d] fp16 against the compressed caches -> [B, Hq, Sq, d]
    fp16 (attention_kernel.py:11-113): GQA by kv head h = q head / (Hq /
    Hkv), scale 1/sqrt(d), the QJL correction with jl_matrix when the keys
    carry signs and enable_qjl, zeros for an empty cache. num_kv_heads is
    taken from the caches, as the reference's working path does."""
    if isinstance(compressed_keys, PQCache):
        from polarquant_kv.attention import compressed_attention_gpu as pq_attention
        return pq_attention(query, compressed_keys, compressed_values, rotation_matrix, jl_matrix=jl_matrix,
                            enable_qjl=enable_qjl, num_kv_heads=num_kv_heads)
    if compressed_keys.seq_len == 0:
        return torch.zeros_like(query)
    return group_attention(query, compressed_keys, compressed_values, rotation_matrix, jl_matrix, enable_qjl,
                           out_dtype=torch.float16)
