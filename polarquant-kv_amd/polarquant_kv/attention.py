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
    kcb, vcb = _codebook_tables(keys, values, mixed, Hkv)
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


def decode_attention_segments(query: torch.Tensor, segments: list, rotation_matrix: torch.Tensor,
                              scale: float | None = None, out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """query [B, Hq, d] against the tokens of several (keys, values) cache
    pairs at once (one softmax over all of them; each pair of uniform widths,
    no QJL) -> out [B, Hq, d]. Segments with no valid tokens are skipped."""
    if query.dim() != 3:
        raise ValueError(f"query must be [B, Hq, d], got {tuple(query.shape)}")
    if not segments:
        raise ValueError("at least one segment is required")
    B, Hq, d = query.shape
    Hkv = None
    for kc, vc in segments:
        if kc.mixed or vc.mixed:
            raise ValueError("segments take caches of one width each")
        h = check_shapes(B, Hq, d, kc, vc, rotation_matrix)
        if Hkv is not None and h != Hkv:
            raise ValueError("every segment must have the same kv heads")
        Hkv = h
    _lib.require_device(query, rotation_matrix)
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    out_dtype = query.dtype if out_dtype is None else out_dtype
    q = query.contiguous()
    R = rotation_matrix.to(torch.float32).contiguous()
    out = torch.empty(B, Hq, d, dtype=out_dtype, device=q.device)
    lib = _lib.lib()
    n = len(segments)
    S = _lib.int_array([kc.seq_len for kc, _ in segments])
    S_max = _lib.int_array([kc.max_seq_len for kc, _ in segments])
    need = lib.pqkv_decode_segments_workspace_bytes(B, Hq, Hkv, n, S, d)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    kcb = [kc.codebooks.to(torch.float32).contiguous() for kc, _ in segments]
    vcb = [vc.codebooks.to(torch.float32).contiguous() for _, vc in segments]
    _lib.check(lib.pqkv_decode_attn_segments(
        q.data_ptr(), _lib.dtype_code(q.dtype), R.data_ptr(), n,
        _lib.ptr_array([kc.blocks for kc, _ in segments]), _lib.ptr_array([vc.blocks for _, vc in segments]),
        _lib.ptr_array(kcb), _lib.ptr_array(vcb),
        _lib.int_array([kc.n_bits for kc, _ in segments]), _lib.int_array([vc.n_bits for _, vc in segments]),
        S, S_max, B, Hq, Hkv, d, scale, out.data_ptr(), _lib.dtype_code(out_dtype), ws.data_ptr(), ws.numel(),
        _lib.stream_of(q)))
    return out


def prefill_attention(query: torch.Tensor, keys: PQCache, values: PQCache, rotation_matrix: torch.Tensor,
                      q_start: int, causal: bool = True, scale: float | None = None,
                      out_dtype: torch.dtype | None = None, jl_rot: torch.Tensor | None = None) -> torch.Tensor:
    """query [B, Hq, Sq, d] at absolute positions q_start.. against caches that
    already hold them -> out [B, Hq, Sq, d]. Any widths (per-head maps
    included); jl_rot = P R^T adds the QJL correction to every query token."""
    if query.dim() != 4:
        raise ValueError(f"query must be [B, Hq, Sq, d], got {tuple(query.shape)}")
    B, Hq, Sq, d = query.shape
    Hkv = check_shapes(B, Hq, d, keys, values, rotation_matrix)
    _lib.require_device(query, rotation_matrix, jl_rot)
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    out_dtype = query.dtype if out_dtype is None else out_dtype
    q = query.contiguous()
    R = rotation_matrix.to(torch.float32).contiguous()
    out = torch.empty(B, Hq, Sq, d, dtype=out_dtype, device=q.device)
    lib = _lib.lib()
    S = keys.seq_len
    need = lib.pqkv_prefill_workspace_bytes(B, Hq, Hkv, Sq, max(S, 1), d)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
    mixed = keys.mixed or values.mixed
    kbits = _lib.int_array(keys.head_bits()) if mixed else None
    vbits = _lib.int_array(values.head_bits()) if mixed else None
    kcb, vcb = _codebook_tables(keys, values, mixed, Hkv)
    qjl = keys.qjl_signs if jl_rot is not None else None
    if jl_rot is not None and qjl is None:
        raise ValueError("QJL correction requested but the key cache has no signs")
    P = None if jl_rot is None else jl_rot.to(torch.float32).contiguous()
    _lib.check(lib.pqkv_prefill_attn(
        q.data_ptr(), _lib.dtype_code(q.dtype), R.data_ptr(), keys.blocks.data_ptr(), values.blocks.data_ptr(),
        kcb.data_ptr(), vcb.data_ptr(), keys.head_bits()[0], values.head_bits()[0], kbits, vbits,
        _lib.ptr(qjl), _lib.ptr(P), d if P is not None else 0, B, Hq, Hkv, Sq, q_start, S, keys.max_seq_len, d,
        scale, int(causal), out.data_ptr(), _lib.dtype_code(out_dtype), ws.data_ptr(), ws.numel(),
        _lib.stream_of(q)))
    return out


def _codebook_tables(keys: PQCache, values: PQCache, mixed: bool, Hkv: int):
    """The codebook pointers the kernels take: one [16] table each, or per-head
    [Hkv, 16] tables with mixed widths."""
    kcb = keys.codebooks if not mixed or keys.codebooks.dim() == 2 else keys.codebooks.expand(Hkv, 16)
    vcb = values.codebooks if not mixed or values.codebooks.dim() == 2 else values.codebooks.expand(Hkv, 16)
    return kcb.contiguous(), vcb.contiguous()


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
    start = compressed_keys.seq_len - Sq if q_start is None else q_start
    return prefill_attention(query, compressed_keys, compressed_values, rotation_matrix, start, causal=causal,
                             out_dtype=torch.float16, jl_rot=jl_rot)


# ---------------------------------------------------------------------------
# The reference's array-level API (python/polarquant_kv/attention.py)
# ---------------------------------------------------------------------------

def _softmax_np(x):
    import numpy as np
    e = np.exp(x - np.max(x, axis=-1, keepdims=True))
    return e / np.sum(e, axis=-1, keepdims=True)


def standard_attention(query, key, value, num_kv_heads: int | None = None):
    """Uncompressed attention, the reference's baseline
    (python/polarquant_kv/attention.py:20-71): 2-D query (n_q, d) against
    key / value (seq, d), or 3-D GQA query (n_heads, seq_q, d) against
    (n_kv_heads, seq, d); scale 1/sqrt(d), no mask, float32 result, zeros for
    an empty sequence. numpy arrays are computed on the host exactly as the
    reference does; torch tensors on their device in fp32."""
    import numpy as np
    if isinstance(query, torch.Tensor):
        return _standard_attention_torch(query, key, value, num_kv_heads)
    if query.ndim == 2 and key.ndim == 2:
        if key.shape[0] == 0:
            return np.zeros((query.shape[0], query.shape[-1]), dtype=np.float32)
        w = _softmax_np(query @ key.T / np.sqrt(query.shape[-1]))
        return (w @ value).astype(np.float32)
    if query.ndim == 3 and key.ndim == 3:
        hq, hkv = query.shape[0], key.shape[0]
        if num_kv_heads is not None and hkv != num_kv_heads:
            raise ValueError(f"key heads {hkv} != num_kv_heads {num_kv_heads}")
        rep = hq // hkv
        out = np.zeros_like(query, dtype=np.float32)
        for h in range(hq):
            out[h] = standard_attention(query[h], key[h // rep], value[h // rep])
        return out
    raise ValueError(f"unsupported shapes: query {query.shape}, key {key.shape}")


def _standard_attention_torch(query, key, value, num_kv_heads):
    if query.dim() == 2 and key.dim() == 2:
        query, key, value = query[None], key[None], value[None]
        return _standard_attention_torch(query, key, value, None)[0]
    if query.dim() != 3 or key.dim() != 3:
        raise ValueError(f"unsupported shapes: query {tuple(query.shape)}, key {tuple(key.shape)}")
    hq, hkv, d = query.shape[0], key.shape[0], query.shape[-1]
    if num_kv_heads is not None and hkv != num_kv_heads:
        raise ValueError(f"key heads {hkv} != num_kv_heads {num_kv_heads}")
    if key.shape[1] == 0:
        return torch.zeros(query.shape, dtype=torch.float32, device=query.device)
    rep = hq // hkv
    k = key.float().repeat_interleave(rep, 0)
    v = value.float().repeat_interleave(rep, 0)
    s = torch.matmul(query.float(), k.transpose(-1, -2).contiguous()) / math.sqrt(d)
    return torch.matmul(torch.softmax(s, -1), v)


def compressed_attention(query, key, value, rotation_matrix, jl_matrix=None, n_bits: int = 4,
                         group_size: int = 32, enable_qjl: bool = True, num_kv_heads: int | None = None,
                         return_scores: bool = False):
    """The reference's compressed attention on arrays
    (python/polarquant_kv/attention.py:83-191): compress key and value, then
    attend on the compressed data, with the QJL score correction when a JL
    matrix is given. Shapes as standard_attention; returns float32 numpy
    (or {"output", "scores"} for 2-D input with return_scores).

    Here the key and value go to the GPU, are encoded in the codebook format
    (block_pq4 / block_pq2, Lloyd-Max centroids, the north-star format; the
    reference's CPU function uses its per-group min/scale quantiser) by the
    HIP encoder, and attended by the HIP decode (one query token) or prefill
    (several, no mask) kernels. group_size is checked as the reference
    checks it."""
    import numpy as np
    from . import quantizer
    from .qjl import rotated_jl_matrix

    q_np, k_np, v_np = (np.asarray(a) for a in (query, key, value))
    two_d = q_np.ndim == 2 and k_np.ndim == 2
    if two_d:
        q_np, k_np, v_np = q_np[None], k_np[None], v_np[None]
    elif not (q_np.ndim == 3 and k_np.ndim == 3):
        raise ValueError(f"unsupported shapes: query {q_np.shape}, key {k_np.shape}")
    hq, sq, d = q_np.shape
    hkv, S = k_np.shape[0], k_np.shape[1]
    if num_kv_heads is not None and hkv != num_kv_heads:
        raise ValueError(f"key heads {hkv} != num_kv_heads {num_kv_heads}")
    quantizer._validate_params(n_bits, group_size, d)
    if S == 0:
        out = np.zeros((hq, sq, d), dtype=np.float32)
        if two_d:
            out = out[0]
            if return_scores:
                return {"output": out, "scores": np.empty((sq, 0), dtype=np.float32)}
        return out
    dev = torch.device("cuda", torch.cuda.current_device()) if torch.cuda.is_available() else None
    if dev is None:
        raise RuntimeError("compressed_attention runs on the GPU (the hot path has no CPU fallback)")
    R = torch.from_numpy(np.asarray(rotation_matrix, np.float32)).to(dev)
    kt = torch.from_numpy(np.ascontiguousarray(k_np, np.float32))[None].to(dev)
    vt = torch.from_numpy(np.ascontiguousarray(v_np, np.float32))[None].to(dev)
    qt = torch.from_numpy(np.ascontiguousarray(q_np, np.float32))[None].to(dev)
    use_qjl = enable_qjl and jl_matrix is not None
    P_rot = rotated_jl_matrix(jl_matrix, np.asarray(rotation_matrix), dev) if use_qjl else None
    kc = quantizer.compress_pq(kt, R, n_bits, jl_rot=P_rot)
    vc = quantizer.compress_pq(vt, R, n_bits)
    if sq == 1:
        out = decode_attention(qt[:, :, 0], kc, vc, R, jl_rot=P_rot, out_dtype=torch.float32)[:, :, None]
    else:
        out = prefill_attention(qt, kc, vc, R, q_start=0, causal=False, jl_rot=P_rot, out_dtype=torch.float32)
    out = out[0].cpu().numpy()
    if not two_d:
        return out
    out = out[0]
    if not return_scores:
        return out
    # scores s = q_rot . k_hat_rot / sqrt(d) (+ the QJL term), from the
    # rotated-space reconstruction of the same cache
    Kr = quantizer.dequantize(kc, None, torch.float32)[0, 0]                # [S, d] rotated
    from .rotation import rotate
    q_rot = rotate(qt[0, 0].contiguous(), R)                                # [sq, d]
    s = q_rot @ Kr.T
    if use_qjl:
        from .qjl import bit_unpack
        signs = bit_unpack(kc.qjl_signs[0, 0, :S], d).to(torch.float32) * 2 - 1
        pq = rotate(q_rot.contiguous(), P_rot) / d
        rk = (Kr.norm(dim=-1) > 0).to(torch.float32)
        s = s + (pq @ signs.T) * rk
    return {"output": out, "scores": (s / math.sqrt(d)).cpu().numpy()}
