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
from .types import PagedPQCache, PQCache, vector_bytes


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


def check_paged(B: int, Hq: int, d: int, keys: PagedPQCache, values: PagedPQCache, rotation_matrix=None) -> int:
    """check_shapes for paged caches: the same geometry, uniform and equal
    widths, one page size, pages covering seq_len. Returns Hkv."""
    if not isinstance(keys, PagedPQCache) or not isinstance(values, PagedPQCache):
        raise ValueError("keys and values must both be paged caches, or both PQCache")
    Hkv = keys.num_heads
    if keys.head_dim != d or values.head_dim != d:
        raise ValueError(f"head_dim: query {d}, keys {keys.head_dim}, values {values.head_dim}")
    if values.num_heads != Hkv or keys.batch != B or values.batch != B:
        raise ValueError("keys and values must match the query's batch and each other's heads")
    if keys.seq_len != values.seq_len:
        raise ValueError("keys and values hold different numbers of positions")
    if keys.n_bits != values.n_bits:
        raise ValueError("paged caches take keys and values of one width")
    if keys.page_tokens != values.page_tokens:
        raise ValueError("keys and values must share page_tokens")
    for c in (keys, values):
        if c.capacity < c.seq_len:
            raise ValueError("paged cache holds fewer pages than its seq_len needs")
    # one table width for both (the kernels take one row stride)
    width = max(keys.max_pages, values.max_pages)
    keys._widen(width)
    values._widen(width)
    if Hq % Hkv:
        raise ValueError(f"Hq={Hq} is not a multiple of Hkv={Hkv}")
    if rotation_matrix is not None and tuple(rotation_matrix.shape) != (d, d):
        raise ValueError(f"rotation matrix must be ({d}, {d}), got {tuple(rotation_matrix.shape)}")
    return Hkv


def decode_attention(query: torch.Tensor, keys: PQCache, values: PQCache, rotation_matrix: torch.Tensor,
                     scale: float | None = None, jl_rot: torch.Tensor | None = None,
                     out_dtype: torch.dtype | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """query [B, Hq, d] (original space) -> out [B, Hq, d] (original space).
    keys / values: PQCache, or PagedPQCache (pqkv_decode_attn_paged)."""
    if query.dim() != 3:
        raise ValueError(f"query must be [B, Hq, d], got {tuple(query.shape)}")
    B, Hq, d = query.shape
    if isinstance(keys, PagedPQCache) or isinstance(values, PagedPQCache):
        return _decode_paged(query, keys, values, rotation_matrix, scale, jl_rot, out_dtype, workspace)
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


def _decode_paged(query, keys, values, rotation_matrix, scale, jl_rot, out_dtype, workspace):
    B, Hq, d = query.shape
    Hkv = check_paged(B, Hq, d, keys, values, rotation_matrix)
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
    if jl_rot is not None and keys.sign_table is None:
        raise ValueError("QJL correction requested but the key cache has no signs")
    P = None if jl_rot is None else jl_rot.to(torch.float32).contiguous()
    _lib.check(lib.pqkv_decode_attn_paged(
        q.data_ptr(), _lib.dtype_code(q.dtype), R.data_ptr(), keys.table.data_ptr(), values.table.data_ptr(),
        keys.page_tokens, keys.max_pages, keys.codebooks.data_ptr(),
        values.codebooks.data_ptr(), keys.n_bits, keys.sign_table.data_ptr() if P is not None else None,
        _lib.ptr(P), d if P is not None else 0, B, Hq, Hkv, S, d, scale, out.data_ptr(), _lib.dtype_code(out_dtype),
        workspace.data_ptr(), workspace.numel(), _lib.stream_of(q)))
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
    if isinstance(keys, PagedPQCache) or isinstance(values, PagedPQCache):
        return _prefill_paged(query, keys, values, rotation_matrix, q_start, causal, scale, out_dtype, jl_rot)
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


def _prefill_paged(query, keys, values, rotation_matrix, q_start, causal, scale, out_dtype, jl_rot):
    B, Hq, Sq, d = query.shape
    Hkv = check_paged(B, Hq, d, keys, values, rotation_matrix)
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
    if jl_rot is not None and keys.sign_table is None:
        raise ValueError("QJL correction requested but the key cache has no signs")
    P = None if jl_rot is None else jl_rot.to(torch.float32).contiguous()
    _lib.check(lib.pqkv_prefill_attn_paged(
        q.data_ptr(), _lib.dtype_code(q.dtype), R.data_ptr(), keys.table.data_ptr(), values.table.data_ptr(),
        keys.page_tokens, keys.max_pages, keys.codebooks.data_ptr(),
        values.codebooks.data_ptr(), keys.n_bits, keys.sign_table.data_ptr() if P is not None else None,
        _lib.ptr(P), d if P is not None else 0, B, Hq, Hkv, Sq, q_start, S, d, scale, int(causal), out.data_ptr(),
        _lib.dtype_code(out_dtype), ws.data_ptr(), ws.numel(), _lib.stream_of(q)))
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
    (python/polarquant_kv/attention.py:83-191), in its format and semantics:
    every key and value is compressed by the group (min / scale) quantizer
    (quantizer.compress: fp64 rotation, fp32 radius, per-group min / scale,
    one byte per code), scores are q . k_hat / sqrt(d) with k_hat the
    decompressed key, plus, with a JL matrix, (1/m) sum_i (2 s_i - 1) (P q)_i
    / sqrt(d) for the signs of P (k - k_hat) (0 for a zero residual,
    qjl.py:50-51); softmax over all keys; output w v_hat. Shapes as
    standard_attention; float32 numpy out (or {"output", "scores"} for 2-D
    input with return_scores).

    Computed on the GPU: pqkv_group_compress encodes the keys and values,
    pqkv_group_decompress and pqkv_qjl_sketch give the QJL signs of the
    original-space residuals, and pqkv_group_attn attends straight on the
    codes (the reference decompresses and runs numpy products)."""
    import numpy as np
    from . import _lib as L
    from . import quantizer

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
    lib = L.lib()
    ng = -(-d // group_size)
    dpad = ng * group_size
    R64 = torch.from_numpy(np.ascontiguousarray(rotation_matrix, np.float64)).to(dev)
    R32 = R64.to(torch.float32)

    def to_dev(a):
        a = np.ascontiguousarray(a if a.dtype in (np.float16, np.float32) else a.astype(np.float32))
        return torch.from_numpy(a).to(dev)

    kt, vt, qt = to_dev(k_np), to_dev(v_np), to_dev(q_np)
    n = hkv * S
    stream = L.stream_of(kt)
    fields = []
    for x in (kt, vt):
        r = torch.empty(n, dtype=torch.float32, device=dev)
        c = torch.empty(n, dpad, dtype=torch.uint8, device=dev)
        lo = torch.empty(n, ng, dtype=torch.float32, device=dev)
        sc = torch.empty(n, ng, dtype=torch.float32, device=dev)
        L.check(lib.pqkv_group_compress(x.data_ptr(), L.dtype_code(x.dtype), R64.data_ptr(), n, d, n_bits, group_size,
                                        r.data_ptr(), c.data_ptr(), lo.data_ptr(), sc.data_ptr(), stream))
        fields.append((r, c, lo, sc))
    use_qjl = enable_qjl and jl_matrix is not None
    signs = norms = P32 = k_hat = None
    m = 0
    if use_qjl or return_scores:
        r, c, lo, sc = fields[0]
        k_hat = torch.empty(n, d, dtype=torch.float32, device=dev)
        L.check(lib.pqkv_group_decompress(r.data_ptr(), c.data_ptr(), lo.data_ptr(), sc.data_ptr(), R64.data_ptr(),
                                          n, d, group_size, k_hat.data_ptr(), stream))
    if use_qjl:
        P64 = torch.from_numpy(np.ascontiguousarray(jl_matrix, np.float64)).to(dev)
        m = P64.shape[0]
        P32 = P64.to(torch.float32).contiguous()
        signs = torch.empty(n, (m + 7) // 8, dtype=torch.uint8, device=dev)
        norms = torch.empty(n, dtype=torch.float32, device=dev)
        L.check(lib.pqkv_qjl_sketch(kt.data_ptr(), L.dtype_code(kt.dtype), k_hat.data_ptr(),
                                    P64.t().contiguous().data_ptr(), n, d, m, signs.data_ptr(), norms.data_ptr(),
                                    L.F32, stream))
    (kr, kc, klo, ksc), (vr, vc, vlo, vsc) = fields
    rows = hq * sq
    out = torch.empty(rows, d, dtype=torch.float32, device=dev)
    ws = torch.empty(lib.pqkv_group_attn_workspace_bytes(1, rows, hkv, S, d, group_size, m), dtype=torch.uint8,
                     device=dev)
    # one byte per code: the attention reads the codes as 8-bit storage
    L.check(lib.pqkv_group_attn(qt.data_ptr(), L.dtype_code(qt.dtype), R32.data_ptr(), L.ptr(P32), m, kc.data_ptr(),
                                kr.data_ptr(), klo.data_ptr(), ksc.data_ptr(), vc.data_ptr(), vr.data_ptr(),
                                vlo.data_ptr(), vsc.data_ptr(), L.ptr(signs), L.ptr(norms), 8, L.F32, 1, rows, hkv, S,
                                S, d, group_size, float(d) ** -0.5, out.data_ptr(), L.F32, ws.data_ptr(), ws.numel(),
                                stream))
    res = out.reshape(hq, sq, d).cpu().numpy()
    if not two_d:
        return res
    res = res[0]
    if not return_scores:
        return res
    # the 2-D scores: q . k_hat / sqrt(d) (+ the QJL term), from the same
    # decompressed keys and signs
    q32 = qt[0].float()
    s = q32 @ k_hat.T
    if use_qjl:
        from .qjl import bit_unpack
        sv = bit_unpack(signs, m).to(torch.float32) * 2 - 1
        corr = (q32 @ P32.T) @ sv.T / m
        s = s + torch.where((norms > 1e-30)[None, :], corr, torch.zeros_like(corr))
    return {"output": res, "scores": (s / math.sqrt(d)).cpu().numpy()}
