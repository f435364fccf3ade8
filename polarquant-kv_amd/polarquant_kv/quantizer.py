"""PQ4 / PQ2 encoder and decoder entry points (device tensors only).

compress_pq is the codebook counterpart of the reference's compress_gpu
(src/polarquant_kv_cuda/compress_kernel.py:100-189) and of
turboquant_compress (csrc/flash_turboquant.cu:213-225): rotate, polar split,
nearest Lloyd-Max centroid per coordinate, pack into blocks, plus the optional
QJL key sketch. compress_gpu / decompress_gpu keep the reference's names and
arguments for that format; dequantize is the general decoder. quantize_rotated
is the bit-exact surface on fp32 rotated input. compress / decompress /
compress_batch / decompress_batch are the reference's CPU quantizer API over
its group (min / scale) format, computed on the GPU. All call
libpqkv_hip.so; there is no CPU path.
"""

from __future__ import annotations

import torch

from . import _lib
from .lloyd_max import padded_codebook_torch, stacked_codebooks_torch
from .types import PagedPQCache, PQCache, vector_bytes


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
    """Encode kv [B, H, T, d] (fp16, fp32 or bf16, which the encoder widens
    exactly to fp32; other float types are widened here; device) into a PQ
    cache.

    With `cache`, positions start .. start+T-1 (default: cache.seq_len) are
    written in place and seq_len grows to cover them; otherwise a new cache of
    exactly T positions is returned. jl_rot = P R^T ([d, d] float32) adds the
    QJL sign sketch of each key's residual."""
    _lib.require_device(kv, rotation_matrix, jl_rot)
    if kv.dim() != 4:
        raise ValueError("kv must be [B, H, T, d]")
    B, H, T, d = kv.shape
    if isinstance(cache, PagedPQCache):
        return _compress_paged(kv, rotation_matrix, cache, start, jl_rot)
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
    # the encoders read fp16, fp32 and bf16 (widened exactly to fp32 on the
    # device, as the reference's kv.float() does,
    # src/polarquant_kv_cuda/compress_kernel.py:135); other floating types
    # are widened here
    x = (kv if kv.dtype in (torch.float16, torch.float32, torch.bfloat16) else kv.to(torch.float32)).contiguous()
    x_code = _lib.BF16 if x.dtype == torch.bfloat16 else _lib.dtype_code(x.dtype)
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
        _lib.check(lib.pqkv_encode(x.data_ptr(), x_code, T * d, R.data_ptr(),
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
            _lib.check(lib.pqkv_encode(xq, x_code, H * T * d, R.data_ptr(),
                                       cache.codebooks[h].data_ptr(), bits, base, cache.blocks.shape[1], B, T, d,
                                       _lib.ptr(P), d if P is not None else 0, qjl_ptr, qjl_stride, stream))
    cache.seq_len = max(cache.seq_len, start + T)
    return cache


def _compress_paged(kv, rotation_matrix, cache: PagedPQCache, start, jl_rot):
    """compress_pq into a paged cache: pages are added as needed, then one
    pqkv_encode_paged call writes positions start .. start + T - 1 of every
    stream through the page table."""
    B, H, T, d = kv.shape
    start = cache.seq_len if start is None else int(start)
    if cache.head_dim != d or cache.batch != B or cache.num_heads != H:
        raise ValueError("cache shape does not match kv")
    if start < 0:
        raise ValueError(f"start {start} < 0")
    if jl_rot is not None and cache.sign_table is None:
        raise ValueError("cache was allocated without QJL signs")
    if T == 0:
        return cache
    cache.ensure(start + T)
    x = (kv if kv.dtype in (torch.float16, torch.float32, torch.bfloat16) else kv.to(torch.float32)).contiguous()
    x_code = _lib.BF16 if x.dtype == torch.bfloat16 else _lib.dtype_code(x.dtype)
    R = rotation_matrix.to(torch.float32).contiguous()
    P = None if jl_rot is None else jl_rot.to(torch.float32).contiguous()
    _lib.check(_lib.lib().pqkv_encode_paged(
        x.data_ptr(), x_code, T * d, R.data_ptr(), cache.codebooks.data_ptr(), cache.n_bits,
        cache.table.data_ptr(), cache.page_tokens, cache.max_pages, start, B * H, T, d, _lib.ptr(P),
        d if P is not None else 0, cache.sign_table.data_ptr() if P is not None else None, _lib.stream_of(x)))
    cache.seq_len = max(cache.seq_len, start + T)
    return cache


def allocate_paged_cache(batch: int, num_heads: int, head_dim: int, n_bits: int = 4, device="cuda",
                         page_tokens: int = 256, jl_dim: int = 0, codebooks=None) -> PagedPQCache:
    """Empty paged cache (no pages yet; compress_pq adds them)."""
    if codebooks is None:
        codebooks = padded_codebook_torch(head_dim, n_bits, device)
    return PagedPQCache(batch, num_heads, head_dim, n_bits, codebooks, device, page_tokens=page_tokens,
                        jl_dim=jl_dim)


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
    rotated-space reconstruction (R = I, exact). A paged cache is gathered
    into one array first."""
    if isinstance(cache, PagedPQCache):
        cache = cache.to_contiguous(positions)
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


# ---------------------------------------------------------------- group format
#
# The reference's CPU quantizer API (python/polarquant_kv/quantizer.py:88-222:
# compress, decompress, compress_batch, decompress_batch) over the group
# (min / scale) format, computed by pqkv_group_compress / pqkv_group_decompress
# on the GPU. Host numpy in, host numpy out, as there; the arithmetic runs on
# the device only.

def _group_device() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("the group quantizer runs on the GPU (no CPU fallback) and no device is available")
    return torch.device("cuda", torch.cuda.current_device())


def _rotation64(rotation_matrix, device) -> torch.Tensor:
    if torch.is_tensor(rotation_matrix):
        return rotation_matrix.to(device=device, dtype=torch.float64).contiguous()
    import numpy as np
    return torch.from_numpy(np.ascontiguousarray(rotation_matrix, dtype=np.float64)).to(device)


def group_compress_arrays(x, rotation_matrix, n_bits: int = 4, group_size: int = 32):
    """x [N, d] (host or device; fp16 input stays fp16, anything else is
    taken as fp32) -> (radius [N] f32, codes [N, d_pad] u8, mins [N, ng] f32,
    scales [N, ng] f32) as host numpy arrays."""
    import numpy as np
    dev = _group_device()
    if torch.is_tensor(x):
        xt = x.to(dev)
        if xt.dtype != torch.float16:
            xt = xt.to(torch.float32)
    else:
        arr = np.asarray(x)
        xt = torch.from_numpy(np.ascontiguousarray(arr if arr.dtype == np.float16 else arr.astype(np.float32))).to(dev)
    if xt.dim() != 2:
        raise ValueError("x must be [N, d]")
    xt = xt.contiguous()
    n, d = xt.shape
    _validate_params(n_bits, group_size, d)
    if d > 256:
        raise ValueError(f"the GPU group quantizer takes d <= 256, got {d}")
    ng = -(-d // group_size)
    R = _rotation64(rotation_matrix, dev)
    if R.shape != (d, d):
        raise ValueError(f"rotation_matrix must be [{d}, {d}], got {tuple(R.shape)}")
    radius = torch.empty(n, dtype=torch.float32, device=dev)
    codes = torch.empty(n, ng * group_size, dtype=torch.uint8, device=dev)
    mins = torch.empty(n, ng, dtype=torch.float32, device=dev)
    scales = torch.empty(n, ng, dtype=torch.float32, device=dev)
    _lib.check(_lib.lib().pqkv_group_compress(xt.data_ptr(), _lib.dtype_code(xt.dtype), R.data_ptr(), n, d, n_bits,
                                              group_size, radius.data_ptr(), codes.data_ptr(), mins.data_ptr(),
                                              scales.data_ptr(), _lib.stream_of(xt)))
    return radius.cpu().numpy(), codes.cpu().numpy(), mins.cpu().numpy(), scales.cpu().numpy()


def group_decompress_arrays(radius, codes, mins, scales, rotation_matrix, d: int, group_size: int):
    """Inverse of group_compress_arrays: host arrays -> [N, d] float32 numpy."""
    import numpy as np
    dev = _group_device()
    r = torch.from_numpy(np.ascontiguousarray(radius, dtype=np.float32).reshape(-1)).to(dev)
    n = r.numel()
    c = torch.from_numpy(np.ascontiguousarray(codes, dtype=np.uint8).reshape(n, -1)).to(dev)
    lo = torch.from_numpy(np.ascontiguousarray(mins, dtype=np.float32).reshape(n, -1)).to(dev)
    sc = torch.from_numpy(np.ascontiguousarray(scales, dtype=np.float32).reshape(n, -1)).to(dev)
    ng = -(-d // group_size)
    if c.shape[1] != ng * group_size or lo.shape[1] != ng or sc.shape[1] != ng:
        raise ValueError("codes / mins / scales do not match d and group_size")
    R = _rotation64(rotation_matrix, dev)
    out = torch.empty(n, d, dtype=torch.float32, device=dev)
    _lib.check(_lib.lib().pqkv_group_decompress(r.data_ptr(), c.data_ptr(), lo.data_ptr(), sc.data_ptr(), R.data_ptr(),
                                                n, d, group_size, out.data_ptr(), _lib.stream_of(out)))
    return out.cpu().numpy()


def compress(v, rotation_matrix, n_bits: int = 4, group_size: int = 32):
    """One vector v [d] -> CompressedKV (python/polarquant_kv/quantizer.py:88-134):
    rotate, radius, direction, per-group min / scale codes."""
    import numpy as np
    from .types import CompressedKV
    arr = np.asarray(v)
    if arr.ndim != 1:
        raise ValueError(f"compress takes one vector [d], got shape {arr.shape} (compress_batch takes batches)")
    _validate_params(n_bits, group_size, arr.shape[-1])
    r, c, lo, sc = group_compress_arrays(arr[None], rotation_matrix, n_bits, group_size)
    return CompressedKV(radius=np.float32(r[0]), quantized_direction=c[0], group_mins=lo[0], group_scales=sc[0],
                        n_bits=n_bits, group_size=group_size, original_dim=arr.shape[-1])


def decompress(compressed, rotation_matrix):
    """CompressedKV -> the vector [original_dim] float32
    (python/polarquant_kv/quantizer.py:137-158)."""
    out = group_decompress_arrays([compressed.radius], compressed.quantized_direction[None],
                                  compressed.group_mins[None], compressed.group_scales[None], rotation_matrix,
                                  compressed.original_dim, compressed.group_size)
    return out[0]


def compress_batch(kv, rotation_matrix, n_bits: int = 4, group_size: int = 32):
    """kv [batch, num_heads, seq_len, head_dim] -> nested lists [b][h][s] of
    CompressedKV, all vectors in one GPU call; an empty kv gives
    {"empty": True, "shape": kv.shape} (python/polarquant_kv/quantizer.py:161-193)."""
    import logging
    import numpy as np
    from .types import CompressedKV
    from .utils import check_memory_warning, estimate_memory_bytes
    arr = np.asarray(kv)
    if arr.size == 0:
        return {"empty": True, "shape": arr.shape}
    B, H, S, d = arr.shape
    est = estimate_memory_bytes(B, H, S, d, n_bits, group_size, jl_dim=0)
    if check_memory_warning(est):
        logging.getLogger(__name__).warning("estimated memory %.2f GB exceeds 80%% of the available memory",
                                            est / 1e9)
    r, c, lo, sc = group_compress_arrays(arr.reshape(-1, d), rotation_matrix, n_bits, group_size)
    out, i = [], 0
    for _b in range(B):
        heads = []
        for _h in range(H):
            seq = []
            for _s in range(S):
                seq.append(CompressedKV(radius=np.float32(r[i]), quantized_direction=c[i], group_mins=lo[i],
                                        group_scales=sc[i], n_bits=n_bits, group_size=group_size, original_dim=d))
                i += 1
            heads.append(seq)
        out.append(heads)
    return out


def decompress_batch(compressed_list, rotation_matrix):
    """Nested lists from compress_batch -> [batch, num_heads, seq_len, head_dim]
    float32 (python/polarquant_kv/quantizer.py:196-222)."""
    import numpy as np
    if isinstance(compressed_list, dict) and compressed_list.get("empty"):
        return np.empty(compressed_list["shape"], dtype=np.float32)
    if not compressed_list:
        return np.empty((0,), dtype=np.float32)
    B, H = len(compressed_list), len(compressed_list[0])
    S = len(compressed_list[0][0]) if H else 0
    if S == 0:
        return np.zeros((B, H, 0, 0), dtype=np.float32)
    flat = [c for heads in compressed_list for seq in heads for c in seq]
    d, gs = flat[0].original_dim, flat[0].group_size
    out = group_decompress_arrays(np.array([c.radius for c in flat], np.float32),
                                  np.stack([c.quantized_direction for c in flat]),
                                  np.stack([c.group_mins for c in flat]), np.stack([c.group_scales for c in flat]),
                                  rotation_matrix, d, gs)
    return out.reshape(B, H, S, d)
