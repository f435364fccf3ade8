"""Attention on the compressed cache (device tensors only).

compressed_attention_gpu keeps the signature of the reference's
src/polarquant_kv_cuda/attention_kernel.py:11-19 and its semantics
(:74-113): q-head h reads kv-head h // (Hq/Hkv), scores q.k/sqrt(d) plus the
QJL correction times the same scale, softmax, weighted sum of values, fp16
result; an empty cache gives zeros (:38-39). The keys and values are PQCache
objects and the work is done by libpqkv_hip.so: one query token per sequence
runs the split-K decode kernel (pqkv_decode_attn); several run chunked
prefill (pqkv_prefill_attn) with an optional causal rule.
"""

from __future__ import annotations

import math

import torch

from . import _lib
from .types import PQCache, vector_bytes


def _rotated_p(jl_matrix, rotation_matrix, device):
    from .qjl import rotated_jl_matrix
    return rotated_jl_matrix(jl_matrix, rotation_matrix, device)


def check_shapes(B: int, Hq: int, d: int, keys: PQCache, values: PQCache, rotation_matrix=None) -> int:
    """Host-side agreement checks shared by decode and prefill, run before
    any launch (the kernels trust these sizes when they address the caches).
    Returns Hkv."""
    Hkv = keys.num_heads
    if keys.head_dim != d or values.head_dim != d:
        raise ValueError(f"head_dim: query {d}, keys {keys.head_dim}, values {values.head_dim}")
    if values.num_heads != Hkv:
        raise ValueError(f"kv heads: keys {Hkv}, values {values.num_heads}")
    if keys.batch != B or values.batch != B:
        raise ValueError(f"batch: query {B}, keys {keys.batch}, values {values.batch}")
    if keys.seq_len != values.seq_len:
        raise ValueError("keys and values hold different numbers of positions")
    if keys.max_seq_len != values.max_seq_len:
        raise ValueError("keys and values must share max_seq_len")
    if not 0 <= keys.seq_len <= keys.max_seq_len:
        raise ValueError(f"seq_len {keys.seq_len} outside 0..{keys.max_seq_len}")
    if Hq % Hkv:
        raise ValueError(f"Hq={Hq} is not a multiple of Hkv={Hkv}")
    if rotation_matrix is not None and tuple(rotation_matrix.shape) != (d, d):
        raise ValueError(f"rotation matrix must be ({d}, {d}), got {tuple(rotation_matrix.shape)}")
    for name, c in (("keys", keys), ("values", values)):
        per_batch = (sum(c.max_seq_len * vector_bytes(d, b) for b in c.head_bits()))
        if c.blocks.numel() < B * per_batch:
            raise ValueError(f"{name}: {c.blocks.numel()} cache bytes, the shape needs {B * per_batch}")
    if keys.qjl_signs is not None and keys.qjl_signs.numel() < B * Hkv * keys.max_seq_len * (d // 8):
        raise ValueError("keys: QJL sign array smaller than the cache shape")
    return Hkv


def decode_attention(query: torch.Tensor, keys: PQCache, values: PQCache, rotation_matrix: torch.Tensor,
                     scale: float | None = None, jl_rot: torch.Tensor | None = None,
                     out_dtype: torch.dtype | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """query [B, Hq, d] (original space) -> out [B, Hq, d] (original space)."""
    if query.dim() != 3:
        raise ValueError(f"query must be [B, Hq, d], got {tuple(query.shape)}")
    B, Hq, d = query.shape
    Hkv = check_shapes(B, Hq, d, keys, values, rotation_matrix)
    _lib.require_device(query, rotation_matrix, jl_rot)
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    out_dtype = query.dtype if out_dtype is None else out_dtype
    q = query.contiguous()
    R = rotation_matrix.to(torch.float32).contiguous()
    out = torch.empty(B, Hq, d, dtype=out_dtype, device=q.device)
    lib = _lib.lib()
    S = keys.seq_len
    need = lib.pqkv_decode_workspace_bytes(B, Hq, Hkv, max(S, 1), d)
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    mixed = keys.mixed or values.mixed
    kbits = _lib.int_array(keys.head_bits()) if mixed else None
    vbits = _lib.int_array(values.head_bits()) if mixed else None
    kcb = keys.codebooks if not mixed or keys.codebooks.dim() == 2 else keys.codebooks.expand(Hkv, 16)
    vcb = values.codebooks if not mixed or values.codebooks.dim() == 2 else values.codebooks.expand(Hkv, 16)
    kcb = kcb.contiguous()
    vcb = vcb.contiguous()
    qjl = keys.qjl_signs if jl_rot is not None else None
    if jl_rot is not None and qjl is None:
        raise ValueError("QJL correction requested but the key cache has no signs")
    P = None if jl_rot is None else jl_rot.to(torch.float32).contiguous()
    _lib.check(lib.pqkv_decode_attn(
        q.data_ptr(), _lib.dtype_code(q.dtype), R.data_ptr(), keys.blocks.data_ptr(), values.blocks.data_ptr(),
        kcb.data_ptr(), vcb.data_ptr(), keys.head_bits()[0], values.head_bits()[0], kbits, vbits,
        _lib.ptr(qjl), _lib.ptr(P), d if P is not None else 0, B, Hq, Hkv, S, keys.max_seq_len, d, scale,
        out.data_ptr(), _lib.dtype_code(out_dtype), workspace.data_ptr(), workspace.numel(), _lib.stream_of(q)))
    return out


def prefill_attention(query: torch.Tensor, keys: PQCache, values: PQCache, rotation_matrix: torch.Tensor,
                      q_start: int, causal: bool = True, scale: float | None = None,
                      out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """query [B, Hq, Sq, d] at absolute positions q_start.. against caches that
    already hold them -> out [B, Hq, Sq, d]."""
    if query.dim() != 4:
        raise ValueError(f"query must be [B, Hq, Sq, d], got {tuple(query.shape)}")
    B, Hq, Sq, d = query.shape
    Hkv = check_shapes(B, Hq, d, keys, values, rotation_matrix)
    _lib.require_device(query, rotation_matrix)
    if keys.mixed or values.mixed:
        raise ValueError("prefill supports uniform bit widths")
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    out_dtype = query.dtype if out_dtype is None else out_dtype
    q = query.contiguous()
    R = rotation_matrix.to(torch.float32).contiguous()
    out = torch.empty(B, Hq, Sq, d, dtype=out_dtype, device=q.device)
    lib = _lib.lib()
    S = keys.seq_len
    need = lib.pqkv_prefill_workspace_bytes(B, Hq, Hkv, Sq, max(S, 1), d)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    _lib.check(lib.pqkv_prefill_attn(
        q.data_ptr(), _lib.dtype_code(q.dtype), R.data_ptr(), keys.blocks.data_ptr(), values.blocks.data_ptr(),
        keys.codebooks.data_ptr(), values.codebooks.data_ptr(), keys.n_bits, values.n_bits, B, Hq, Hkv, Sq,
        q_start, S, keys.max_seq_len, d, scale, int(causal), out.data_ptr(), _lib.dtype_code(out_dtype),
        ws.data_ptr(), ws.numel(), _lib.stream_of(q)))
    return out


def compressed_attention_gpu(query: torch.Tensor, compressed_keys: PQCache, compressed_values: PQCache,
                             rotation_matrix: torch.Tensor, jl_matrix=None, enable_qjl: bool = True,
                             num_kv_heads: int | None = None, *, causal: bool = False,
                             q_start: int | None = None) -> torch.Tensor:
    """query [B, Hq, Sq, d] fp16 -> [B, Hq, Sq, d] fp16 (the reference's
    compressed_attention_gpu contract). num_kv_heads, when given, must agree
    with the cache. For Sq > 1 the queries sit at positions q_start ..
    (default: the last Sq positions of the cache)."""
    B, Hq, Sq, d = query.shape
    if num_kv_heads is not None and num_kv_heads != compressed_keys.num_heads:
        raise ValueError("num_kv_heads disagrees with the cache")
    if compressed_keys.seq_len == 0:
        return torch.zeros_like(query)
    jl_rot = None
    if enable_qjl and jl_matrix is not None and compressed_keys.qjl_signs is not None:
        jl_rot = _rotated_p(jl_matrix, rotation_matrix, query.device)
    if Sq == 1:
        return decode_attention(query[:, :, 0, :], compressed_keys, compressed_values, rotation_matrix,
                                jl_rot=jl_rot, out_dtype=torch.float16).unsqueeze(2)
    if jl_rot is not None:
        raise ValueError("QJL correction is supported for single-token decode")
    start = compressed_keys.seq_len - Sq if q_start is None else q_start
    return prefill_attention(query, compressed_keys, compressed_values, rotation_matrix, start, causal=causal,
                             out_dtype=torch.float16)
