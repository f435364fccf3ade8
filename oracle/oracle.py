"""CPU oracle for the PolarQuant-KV hot path.

TEST INFRASTRUCTURE ONLY. Nothing in the product (`polarquant-kv_amd/`) may
import, call or link this module. Only `tests/`, `__graft_entry__.smoke()` and
the `cpu_baseline` leg of `bench.py` use it, and only as the checker (or as the
timed CPU baseline), never as the thing measured on the GPU.

Every function restates the reference algorithm it cites (paths are relative
to the reference tree, hilllief/polarquant-kv). Arithmetic that must be
bit-exact (radius, direction, index, packing) is done in IEEE float32 with
numpy elementwise ops, which on x86-64 never contract or widen, so the order
of operations below is the order of rounding. Attention is computed in
float64 as the textbook formula, which is the oracle the HIP kernels are
held to within the stated tolerance.

Parity pins (what checks each function besides itself), see tests/test_oracle.py:
  lloyd_max_codebook   golden vectors written by the reference itself
                       (tests/golden/codebooks.json), symmetry, Gaussian limit
  rotation_matrix      golden R from the reference (tests/golden/*.npy),
                       orthogonality, seed reproducibility
  jl_matrix            golden P from the reference, N(0,1/m) moments
  quantize_rotated     brute force over all centroids, R=I radius, zero
                       vector, exact r*c inputs, the C restatement (pq_oracle.c)
  pack/unpack          the nibble KAT of scripts/debug_kernel2.py:58-82,
                       crumb order of compress_kernel.py:43-50, round trips
  decode_attention     textbook SDPA on the dequantised cache (torch fp64),
                       lossless-cache special case, GQA by repetition
  prefill_attention    decode_attention row by row (causal rule), SDPA
  qjl_*                closed form of qjl.py:38-57, bit-pack round trip,
                       rotated-space identity P e = (P R^T)(R e)
  group_*              hand-worked codes (round half to even, flat groups,
                       padding), zero vector, the reference tests' cosine
                       thresholds per width (tests/test_quantizer.py:66-82)
  gpu_group_*          hand-worked codes and packing (4-, 2-bit, bytes), the
                       zero vector, the reference tests' round-trip cosine
                       thresholds (tests/cuda/test_compress_decompress.py:
                       66-80), the residual identity e = x - x^ for R = I
  group_attention      textbook SDPA (torch fp64) on the same decompressed
                       caches, the zero-residual guard by hand
  ggml_pq4_*           the ggml fixture tables, the R = I identity with the
                       numpy restatement, lossless heads
  ggml_flash_attn_ext  torch's float64 scaled_dot_product_attention with an
                       additive mask (causal and padding masks), GQA by
                       repetition, the all-masked row
"""

from __future__ import annotations

import math
from functools import lru_cache

import numpy as np

BLOCK = 32                       # coordinates per block_pq4 / block_pq2
PQ4_BLOCK_BYTES = 2 + BLOCK // 2  # {fp16 d; uint8 qs[16]}   README.md:73-78
PQ2_BLOCK_BYTES = 2 + BLOCK // 4  # {fp16 d; uint8 qs[8]}    (build-defined 2-bit twin)


# ---------------------------------------------------------------------------
# L0: codebook, rotation, JL matrix
# ---------------------------------------------------------------------------

@lru_cache(maxsize=None)
def _lloyd_max_cached(dim: int, n_bits: int, n_iterations: int, grid_size: int):
    from scipy.stats import beta as beta_dist

    n_levels = 1 << n_bits
    alpha = (dim - 1) / 2.0
    sigma = 1.0 / np.sqrt(dim)
    x_range = 6 * sigma
    grid = np.linspace(-x_range, x_range, grid_size)
    t = np.clip((grid + 1) / 2, 1e-10, 1 - 1e-10)
    pdf = beta_dist.pdf(t, alpha, alpha) / 2
    pdf = pdf / (pdf.sum() * (grid[1] - grid[0]))
    cent = np.linspace(-x_range, x_range, n_levels)
    bounds = None
    for _ in range(n_iterations):
        bounds = np.zeros(n_levels + 1)
        bounds[0] = -x_range * 2
        bounds[-1] = x_range * 2
        for i in range(1, n_levels):
            bounds[i] = (cent[i - 1] + cent[i]) / 2
        new = np.zeros(n_levels)
        for i in range(n_levels):
            m = (grid >= bounds[i]) & (grid < bounds[i + 1])
            if m.sum() > 0:
                w = pdf[m]
                ws = w.sum()
                new[i] = (grid[m] * w).sum() / ws if ws > 0 else cent[i]
            else:
                new[i] = cent[i]
        cent = new
    return cent.astype(np.float32), bounds.astype(np.float32)


def lloyd_max_codebook(dim: int, n_bits: int, n_iterations: int = 300,
                       grid_size: int = 50000):
    """Lloyd-Max centroids for one rotated unit-vector coordinate.

    Follows src/polarquant_kv_cuda/lloyd_max.py:12-79: Beta((d-1)/2,(d-1)/2)
    on [-1,1] sampled on a 50 000-point grid over +-6/sqrt(d), uniform initial
    centroids, 300 midpoint/centroid iterations; the returned boundaries are
    those of the pre-final centroids (lloyd_max.py:57-61 vs :77).
    Returns (centroids f32[2^b], boundaries f32[2^b+1]).
    """
    c, b = _lloyd_max_cached(int(dim), int(n_bits), int(n_iterations), int(grid_size))
    return c.copy(), b.copy()


def rotation_matrix(d: int, seed: int | None = 42) -> np.ndarray:
    """Haar-random orthogonal R (float64), python/polarquant_kv/rotation.py:7-35."""
    from scipy.stats import ortho_group

    if d == 1:
        rng = np.random.Generator(np.random.PCG64(seed))
        return np.array([[rng.choice([-1.0, 1.0])]], dtype=np.float64)
    rng = np.random.default_rng(seed)
    return ortho_group.rvs(d, random_state=rng).astype(np.float64)


def jl_matrix(m: int, d: int, seed: int | None = None) -> np.ndarray:
    """P ~ N(0, 1/m), shape (m, d), float64: python/polarquant_kv/qjl.py:8-22."""
    rng = np.random.Generator(np.random.PCG64(seed))
    return rng.standard_normal((m, d)).astype(np.float64) / np.sqrt(m)


def rotate(v: np.ndarray, R: np.ndarray) -> np.ndarray:
    """v @ R^T in float64 (rotation.py:38-48)."""
    return np.asarray(v, np.float64) @ np.asarray(R, np.float64).T


def inverse_rotate(v: np.ndarray, R: np.ndarray) -> np.ndarray:
    """v @ R in float64 (rotation.py:51-61)."""
    return np.asarray(v, np.float64) @ np.asarray(R, np.float64)


# ---------------------------------------------------------------------------
# L3 encode: radius, direction, nearest centroid (bit-exact, float32)
# ---------------------------------------------------------------------------

def tree_slots(d: int) -> int:
    """Width of the shared-memory reduction tree used for the radius.

    csrc/flash_turboquant.cu:141-147 reduces blockDim.x = 128 slots; the ggml
    copy uses blockDim = max(D, 128) (integration/polarquant-kv.patch:455-457).
    For power-of-two d that is max(d, 128).
    """
    return max(128, 1 << (int(d) - 1).bit_length())


def radius_f32(x_rot: np.ndarray) -> np.ndarray:
    """fp32 radius with the reference's reduction order.

    flash_turboquant.cu:142-148: buf[t] = rot[t]*rot[t] (0 for t >= D), then
    for s = slots/2 .. 1: buf[t] += buf[t+s] (t < s), r = sqrtf(buf[0]).
    """
    x = np.ascontiguousarray(x_rot, dtype=np.float32)
    n, d = x.shape
    slots = tree_slots(d)
    buf = np.zeros((n, slots), np.float32)
    buf[:, :d] = x * x
    s = slots // 2
    while s > 0:
        buf[:, :s] = buf[:, :s] + buf[:, s:2 * s]
        s //= 2
    return np.sqrt(buf[:, 0])


def nearest_centroid(values: np.ndarray, centroids: np.ndarray) -> np.ndarray:
    """argmin_i |v - c_i| with the first minimum winning (lloyd_max.py:82-90;
    the kernels scan i upward with a strict '<', flash_turboquant.cu:164-171)."""
    v = np.asarray(values, np.float32)
    c = np.asarray(centroids, np.float32)
    best = np.zeros(v.shape, np.uint8)
    bestd = np.full(v.shape, np.float32(1e30), np.float32)
    for i in range(c.shape[0]):
        dist = np.abs(v - c[i])
        better = dist < bestd
        best[better] = i
        bestd = np.where(better, dist, bestd)
    return best


def quantize_rotated(x_rot: np.ndarray, centroids: np.ndarray):
    """Bit-exact surface of the encoder on fp32 rotated input.

    flash_turboquant.cu:141-173 / patch:226-268: radius as radius_f32, then
    dir = rot / r (IEEE fp32 divide) when r > 1e-30 else 0, then
    nearest_centroid. Returns (radius f32[N], idx u8[N, d]).
    """
    x = np.ascontiguousarray(x_rot, dtype=np.float32)
    r = radius_f32(x)
    safe = np.where(r > np.float32(1e-30), r, np.float32(1.0)).astype(np.float32)
    direction = np.where((r > np.float32(1e-30))[:, None], x / safe[:, None],
                         np.float32(0.0)).astype(np.float32)
    return r, nearest_centroid(direction, centroids)


def encode(x: np.ndarray, R: np.ndarray, centroids: np.ndarray):
    """Rotate (float64, rounded to fp32) then quantize_rotated.

    The reference rotates in fp32 (flash_turboquant.cu:132-137); any rotation
    that is not that exact FMA chain only matches it to ~1 ulp, so fused
    encoders are compared through `boundary_margin` (documented tie cases).
    Returns (x_rot f32, radius f32, idx u8).
    """
    xr = rotate(np.asarray(x, np.float64).reshape(-1, R.shape[0]), R).astype(np.float32)
    r, idx = quantize_rotated(xr, centroids)
    return xr, r, idx


def boundary_margin(x_rot: np.ndarray, radius: np.ndarray, centroids: np.ndarray) -> np.ndarray:
    """|dir - nearest decision midpoint| per coordinate (float64), used to
    excuse index differences that sit within rounding distance of a tie."""
    c = np.asarray(centroids, np.float64)
    mids = (c[1:] + c[:-1]) / 2
    r = np.asarray(radius, np.float64)
    d = np.where(r[:, None] > 1e-30, np.asarray(x_rot, np.float64) / np.where(r > 1e-30, r, 1)[:, None], 0.0)
    return np.min(np.abs(d[..., None] - mids), axis=-1)


# ---------------------------------------------------------------------------
# Packing: block_pq4 / block_pq2
# ---------------------------------------------------------------------------

def pack_codes(idx: np.ndarray, n_bits: int) -> np.ndarray:
    """Pack per-coordinate codes along the last axis.

    4-bit: element 2i in the low nibble, 2i+1 in the high nibble
    (flash_turboquant.cu:173, compress_kernel.py:36-41).
    2-bit: v0 | v1<<2 | v2<<4 | v3<<6 (compress_kernel.py:43-50).
    """
    q = np.asarray(idx, np.uint8)
    if n_bits == 4:
        return (q[..., 0::2] | (q[..., 1::2] << 4)).astype(np.uint8)
    if n_bits == 2:
        return (q[..., 0::4] | (q[..., 1::4] << 2) | (q[..., 2::4] << 4)
                | (q[..., 3::4] << 6)).astype(np.uint8)
    raise ValueError(f"n_bits must be 2 or 4, got {n_bits}")


def unpack_codes(packed: np.ndarray, n_bits: int) -> np.ndarray:
    p = np.asarray(packed, np.uint8)
    if n_bits == 4:
        out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), np.uint8)
        out[..., 0::2] = p & 0x0F
        out[..., 1::2] = p >> 4
        return out
    if n_bits == 2:
        out = np.empty(p.shape[:-1] + (p.shape[-1] * 4,), np.uint8)
        for k in range(4):
            out[..., k::4] = (p >> (2 * k)) & 0x3
        return out
    raise ValueError(f"n_bits must be 2 or 4, got {n_bits}")


def block_bytes(n_bits: int) -> int:
    return PQ4_BLOCK_BYTES if n_bits == 4 else PQ2_BLOCK_BYTES


def vector_bytes(d: int, n_bits: int) -> int:
    return (d // BLOCK) * block_bytes(n_bits)


def pack_blocks(radius: np.ndarray, idx: np.ndarray, n_bits: int = 4) -> np.ndarray:
    """Serialise (radius, codes) into block_pq4 (18 B / 32 coords) or
    block_pq2 (10 B / 32 coords). Layout of one block: bytes 0-1 the fp16
    radius of the whole vector (little endian, RNE from fp32), then the packed
    codes of its 32 coordinates (README.md:73-78). Shape (..., d/32*bb).
    Radii above 65504 are stored as 65504, the reference's saturating fp16
    radius (src/polarquant_kv_cuda/compress_kernel.py:178)."""
    idx = np.asarray(idx, np.uint8)
    lead = idx.shape[:-1]
    d = idx.shape[-1]
    nb = d // BLOCK
    bb = block_bytes(n_bits)
    r32 = np.asarray(radius, np.float32)
    # saturated fp16, compress_kernel.py:178: clamp(-65504, 65504).half()
    # (a radius is >= 0; NaN stays NaN)
    r16 = np.where(r32 > np.float32(65504.0), np.float32(65504.0), r32).astype(np.float16).reshape(lead + (1,))
    rbytes = r16.view(np.uint8).reshape(lead + (2,))
    out = np.empty(lead + (nb, bb), np.uint8)
    codes = idx.reshape(lead + (nb, BLOCK))
    out[..., 0:2] = rbytes[..., None, :]
    out[..., 2:] = pack_codes(codes, n_bits)
    return out.reshape(lead + (nb * bb,))


def unpack_blocks(blocks: np.ndarray, d: int, n_bits: int = 4):
    """Inverse of pack_blocks: returns (radius f16 [...], idx u8 [..., d]).
    The radius is read from the first block of each vector."""
    b = np.asarray(blocks, np.uint8)
    lead = b.shape[:-1]
    nb = d // BLOCK
    bb = block_bytes(n_bits)
    bl = b.reshape(lead + (nb, bb))
    r16 = np.ascontiguousarray(bl[..., 0, 0:2]).view(np.float16).reshape(lead)
    idx = unpack_codes(bl[..., 2:], n_bits).reshape(lead + (d,))
    return r16, idx


def dequantize_rotated(blocks: np.ndarray, d: int, centroids: np.ndarray, n_bits: int = 4):
    """Rotated-space reconstruction r16 * c[idx] in float64."""
    r16, idx = unpack_blocks(blocks, d, n_bits)
    c = np.asarray(centroids, np.float32).astype(np.float64)
    return r16.astype(np.float64)[..., None] * c[idx]


# ---------------------------------------------------------------------------
# QJL (keys)
# ---------------------------------------------------------------------------

def bit_pack_lsb(signs: np.ndarray) -> np.ndarray:
    """[..., m] bool -> [..., ceil(m/8)] u8, bit 0 first (qjl_kernel.py:112-124)."""
    s = np.asarray(signs, bool)
    m = s.shape[-1]
    pad = (-m) % 8
    if pad:
        s = np.concatenate([s, np.zeros(s.shape[:-1] + (pad,), bool)], axis=-1)
    g = s.reshape(s.shape[:-1] + (-1, 8)).astype(np.uint8)
    return (g * (1 << np.arange(8, dtype=np.uint8))).sum(-1).astype(np.uint8)


def bit_unpack_lsb(packed: np.ndarray, m: int) -> np.ndarray:
    p = np.asarray(packed, np.uint8)
    bits = (p[..., None] >> np.arange(8, dtype=np.uint8)) & 1
    return bits.reshape(p.shape[:-1] + (-1,))[..., :m].astype(bool)


def qjl_signs_rotated(x_rot: np.ndarray, radius: np.ndarray, idx: np.ndarray,
                      centroids: np.ndarray, P_rot: np.ndarray):
    """Sign sketch of the key residual, computed in the rotated space.

    compress_kernel.py:169-175: e = k - k_hat with k_hat = dir_hat * r (fp32
    radius), signs = (P e >= 0) packed LSB-first. With P_rot = P R^T the same
    projection is P_rot e_rot (e_rot = R e). Returns (packed u8[..., m/8],
    residual norm f64[...]).
    """
    c = np.asarray(centroids, np.float32).astype(np.float64)
    e = np.asarray(x_rot, np.float64) - np.asarray(radius, np.float64)[..., None] * c[idx]
    proj = e @ np.asarray(P_rot, np.float64).T
    return bit_pack_lsb(proj >= 0), np.linalg.norm(e, axis=-1)


def qjl_zero_residual(packed: np.ndarray, m: int) -> np.ndarray:
    """Keys whose residual is zero, as far as the stored sketch tells: a zero
    residual projects to P 0 = 0 >= 0, so every one of its m signs is 1
    (qjl_kernel.py:31, qjl.py:32). The CPU guard returns correction 0 for a
    zero residual (qjl.py:50-51, the reference test AC-3.5 at
    tests/test_qjl.py:139-154); a block cache keeps no residual norm, so the
    all-ones sketch stands for it (a non-zero residual has all signs 1 with
    probability 2^-m). packed [..., ceil(m/8)] -> bool [...]."""
    return np.all(bit_unpack_lsb(np.asarray(packed), m), axis=-1)


def qjl_correction(q: np.ndarray, packed: np.ndarray, P: np.ndarray) -> np.ndarray:
    """(1/m) sum_i (2 s_i - 1) (P q)_i, qjl.py:53-55 / attention_kernel.py:99-106.
    q [..., d] against packed [S, m/8] -> [..., S]."""
    m = P.shape[0]
    s = 2.0 * bit_unpack_lsb(packed, m).astype(np.float64) - 1.0
    qp = np.asarray(q, np.float64) @ np.asarray(P, np.float64).T
    return qp @ s.T / m


# ---------------------------------------------------------------------------
# Attention on the compressed cache (float64)
# ---------------------------------------------------------------------------

def decode_attention(q: np.ndarray, k_blocks: np.ndarray, v_blocks: np.ndarray,
                     R: np.ndarray, k_cb: np.ndarray, v_cb: np.ndarray,
                     seq_len: int | None = None, k_bits=4, v_bits=4,
                     scale: float | None = None, qjl_signs=None, P=None):
    """Single-token attention over a block-encoded cache, in float64.

    q [B, Hq, d] (original space); k_blocks/v_blocks [B, Hkv, S, bytes].
    k_bits / v_bits: int or per-kv-head sequence (mixed 2/4-bit heads).
    Semantics (flash_turboquant.cu:27-105, patch:277-389, attention_kernel.py:
    74-113, benchmark_turboquant.py:102,120): q_rot = q R^T; s_t = scale *
    r_k,t * q_rot . c[idx_t] (+ scale * QJL correction when signs given, with
    correction 0 for a zero residual, i.e. an all-ones sketch, qjl.py:50-51,
    see qjl_zero_residual); w = softmax(s);
    o = (sum_t w_t r_v,t c[vidx_t]) R. GQA: q-head h reads kv-head h // (Hq/Hkv).
    S = 0 gives zeros (attention_kernel.py:38-39).
    """
    q = np.asarray(q, np.float64)
    B, Hq, d = q.shape
    Hkv = k_blocks.shape[1]
    S = k_blocks.shape[2] if seq_len is None else int(seq_len)
    if S == 0:
        return np.zeros((B, Hq, d))
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    kb = [k_bits] * Hkv if np.isscalar(k_bits) else list(k_bits)
    vb = [v_bits] * Hkv if np.isscalar(v_bits) else list(v_bits)
    grp = Hq // Hkv
    q_rot = rotate(q, R)
    out = np.zeros((B, Hq, d))
    for b in range(B):
        for h in range(Hkv):
            kcb = k_cb[h] if isinstance(k_cb, (list, tuple)) else k_cb
            vcb = v_cb[h] if isinstance(v_cb, (list, tuple)) else v_cb
            K = dequantize_rotated(k_blocks[b, h, :S], d, kcb, kb[h])   # [S, d]
            V = dequantize_rotated(v_blocks[b, h, :S], d, vcb, vb[h])
            qs = q_rot[b, h * grp:(h + 1) * grp]                        # [g, d]
            s = (qs @ K.T) * scale
            if qjl_signs is not None and P is not None:
                corr = qjl_correction(q[b, h * grp:(h + 1) * grp], qjl_signs[b, h, :S], P)
                corr = np.where(qjl_zero_residual(qjl_signs[b, h, :S], P.shape[0])[None, :], 0.0, corr)
                s = s + corr * scale
            s = s - s.max(axis=-1, keepdims=True)
            w = np.exp(s)
            w /= w.sum(axis=-1, keepdims=True)
            out[b, h * grp:(h + 1) * grp] = w @ V
    return inverse_rotate(out, R)


def decode_attention_soa(q_rot: np.ndarray, k_packed: np.ndarray, k_radius: np.ndarray,
                         v_packed: np.ndarray, v_radius: np.ndarray, codebook: np.ndarray,
                         n_kv_heads: int, scale: float) -> np.ndarray:
    """The reference's fused attention on its SoA cache, in float64, with the
    fp32 radii as given (integration/polarquant-kv.patch:320-389,
    csrc/flash_turboquant.cu:27-105): q_rot [Hq, d] already rotated;
    k_packed / v_packed [Hkv * S, d/2] (coordinate 2i in the low nibble),
    k_radius / v_radius [Hkv * S] fp32; q-head h reads kv-head
    h // (Hq / Hkv); s_t = scale * r_k,t * q_rot . c[idx_t], w = softmax(s),
    o_rot = sum_t w_t r_v,t c[vidx_t]. Returns the rotated output [Hq, d]."""
    q = np.asarray(q_rot, np.float64)
    Hq, d = q.shape
    S = k_radius.shape[0] // n_kv_heads
    c = np.asarray(codebook, np.float32).astype(np.float64)
    K = np.asarray(k_radius, np.float32).astype(np.float64)[:, None] * c[unpack_codes(k_packed, 4)]
    V = np.asarray(v_radius, np.float32).astype(np.float64)[:, None] * c[unpack_codes(v_packed, 4)]
    K = K.reshape(n_kv_heads, S, d)
    V = V.reshape(n_kv_heads, S, d)
    g = Hq // n_kv_heads
    out = np.zeros((Hq, d))
    for h in range(Hq):
        s = K[h // g] @ q[h] * scale
        w = np.exp(s - s.max())
        out[h] = (w / w.sum()) @ V[h // g]
    return out


def prefill_attention(q: np.ndarray, k_blocks: np.ndarray, v_blocks: np.ndarray,
                      R: np.ndarray, k_cb, v_cb, q_start: int, causal: bool = True,
                      k_bits=4, v_bits=4, scale: float | None = None, qjl_signs=None, P=None):
    """Chunked prefill against an encoded cache that already holds the chunk.

    q [B, Hq, Sq, d]; the cache [B, Hkv, S_total, bytes] holds positions
    0 .. q_start+Sq-1 (append-then-attend, inference/attention.py:59-61).
    Query i of the chunk (absolute position q_start+i) attends to positions
    <= q_start+i when causal, to all S_total positions otherwise. The QJL
    correction (qjl_signs [B, Hkv, S_total, m/8], P) applies to every query
    token, as attention_kernel.py:95-107 does for Sq > 1.
    Computed as one decode_attention per query row.
    """
    q = np.asarray(q, np.float64)
    B, Hq, Sq, d = q.shape
    S_total = k_blocks.shape[2]
    out = np.zeros((B, Hq, Sq, d))
    for i in range(Sq):
        L = q_start + i + 1 if causal else S_total
        out[:, :, i] = decode_attention(q[:, :, i], k_blocks[:, :, :L], v_blocks[:, :, :L],
                                        R, k_cb, v_cb, k_bits=k_bits, v_bits=v_bits,
                                        scale=scale,
                                        qjl_signs=None if qjl_signs is None else qjl_signs[:, :, :L], P=P)
    return out


def sdpa(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float | None = None) -> np.ndarray:
    """Textbook attention in float64: q [..., Sq, d], k/v [..., S, d]."""
    q = np.asarray(q, np.float64)
    d = q.shape[-1]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    s = q @ np.swapaxes(np.asarray(k, np.float64), -1, -2) * scale
    s = s - s.max(axis=-1, keepdims=True)
    w = np.exp(s)
    w /= w.sum(axis=-1, keepdims=True)
    return w @ np.asarray(v, np.float64)


# ---------------------------------------------------------------------------
# Synthetic inputs of the benchmark configurations
# ---------------------------------------------------------------------------

# ---------------------------------------------------------------------------
# Group (min / scale) format of the reference's CPU quantizer
# ---------------------------------------------------------------------------

def group_quantize_direction(u: np.ndarray, n_bits: int, group_size: int):
    """Per-group min / scale codes of a direction u [d] (float32)
    (python/polarquant_kv/quantizer.py:25-66): zero-pad to whole groups;
    scale = (max - min) / levels, 1 for a flat group; codes
    clip(round_half_even((u - min) / scale), 0, levels), 0 in a flat group."""
    d = u.shape[-1]
    ng = math.ceil(d / group_size)
    u = np.concatenate([u.astype(np.float32), np.zeros(ng * group_size - d, np.float32)])
    groups = u.reshape(ng, group_size)
    lo = groups.min(axis=1).astype(np.float32)
    hi = groups.max(axis=1).astype(np.float32)
    levels = (1 << n_bits) - 1
    scales = np.where(hi - lo > 0, (hi - lo) / np.float32(levels), np.float32(1.0)).astype(np.float32)
    codes = np.zeros((ng, group_size), np.uint8)
    for g in range(ng):
        if scales[g] > 0 and hi[g] - lo[g] > 0:
            codes[g] = np.clip(np.round((groups[g] - lo[g]) / scales[g]), 0, levels).astype(np.uint8)
    return codes.reshape(-1), lo, scales


def group_compress(v: np.ndarray, R: np.ndarray, n_bits: int, group_size: int):
    """One vector -> (radius f32, codes, mins, scales)
    (python/polarquant_kv/quantizer.py:88-134; rotation.py:48 rotates in
    fp64 and casts back to fp32)."""
    v32 = np.asarray(v).astype(np.float32)
    y = (v32.astype(np.float64) @ R.T).astype(np.float32)
    r = np.float32(np.linalg.norm(y))
    d = y.shape[-1]
    ng = math.ceil(d / group_size)
    if r < 1e-30:
        return np.float32(0.0), np.zeros(ng * group_size, np.uint8), np.zeros(ng, np.float32), np.ones(ng, np.float32)
    codes, lo, sc = group_quantize_direction((y / r).astype(np.float32), n_bits, group_size)
    return r, codes, lo, sc


def group_decompress(r, codes, lo, sc, R: np.ndarray, d: int, group_size: int) -> np.ndarray:
    """(python/polarquant_kv/quantizer.py:69-85,137-158): u = code * scale +
    min in fp32, the first d values times r, rotated back in fp64."""
    if r < 1e-30:
        return np.zeros(d, np.float32)
    ng = len(lo)
    g = codes[:ng * group_size].reshape(ng, group_size).astype(np.float32)
    g = g * sc.astype(np.float32)[:, None] + lo.astype(np.float32)[:, None]
    y = g.reshape(-1)[:d] * np.float32(r)
    return (y.astype(np.float64) @ R).astype(np.float32)


# ---------------------------------------------------------------------------
# The reference's GPU group format (CompressedKVCacheGPU)
# ---------------------------------------------------------------------------

def gpu_group_store_bits(n_bits: int) -> int:
    """4- and 2-bit codes are packed, every other width keeps one byte per
    code (compress_kernel.py:17-63: 3- and 6-bit "simplified" to bytes)."""
    return 4 if n_bits == 4 else 2 if n_bits == 2 else 8


def gpu_group_pack(codes: np.ndarray, n_bits: int) -> np.ndarray:
    """[..., d_pad] uint8 -> packed rows (compress_kernel.py:17-63): 4-bit
    (high << 4) | low of the pair (2i, 2i + 1); 2-bit v0 | v1<<2 | v2<<4 |
    v3<<6; other widths unchanged."""
    c = np.asarray(codes).astype(np.uint32)
    if n_bits == 4:
        return (c[..., 0::2] | (c[..., 1::2] << 4)).astype(np.uint8)
    if n_bits == 2:
        return (c[..., 0::4] | (c[..., 1::4] << 2) | (c[..., 2::4] << 4) | (c[..., 3::4] << 6)).astype(np.uint8)
    return c.astype(np.uint8)


def gpu_group_unpack(packed: np.ndarray, n_bits: int) -> np.ndarray:
    """Inverse of gpu_group_pack (compress_kernel.py:66-97)."""
    p = np.asarray(packed).astype(np.uint32)
    if n_bits == 4:
        out = np.empty(p.shape[:-1] + (2 * p.shape[-1],), np.uint8)
        out[..., 0::2] = p & 15
        out[..., 1::2] = p >> 4
        return out
    if n_bits == 2:
        out = np.empty(p.shape[:-1] + (4 * p.shape[-1],), np.uint8)
        for k in range(4):
            out[..., k::4] = (p >> (2 * k)) & 3
        return out
    return p.astype(np.uint8)


def gpu_group_quantize(y: np.ndarray, n_bits: int, group_size: int):
    """The quantiser of compress_gpu on rotated vectors y [n, d] float32
    (src/polarquant_kv_cuda/compress_kernel.py:137-163), fp32 elementwise:
    r = |y| (fp32 of the fp64 sum of squares), safe = max(r, 1e-30), u =
    y / safe and 0 where r < 1e-30, zero-padded to whole groups; per group
    lo = min, range = max - lo, s = range / L where range > 0 else 1 (L =
    2^bits - 1); code = round_half_even(clip((u - lo) / s, 0, L)).
    Returns (r, safe, codes [n, d_pad] uint8, lo [n, ng], s [n, ng]), lo and
    s unrounded fp32."""
    y = np.asarray(y, np.float32)
    n, d = y.shape
    ng = math.ceil(d / group_size)
    r = np.sqrt((y.astype(np.float64) ** 2).sum(-1)).astype(np.float32)
    zero = r < np.float32(1e-30)
    safe = np.where(zero, np.float32(1e-30), r).astype(np.float32)
    u = np.zeros((n, ng * group_size), np.float32)
    u[:, :d] = np.where(zero[:, None], np.float32(0.0), y / safe[:, None])
    g = u.reshape(n, ng, group_size)
    lo = g.min(-1)
    rng = (g.max(-1) - lo).astype(np.float32)
    L = np.float32((1 << n_bits) - 1)
    sc = np.where(rng > 0, rng / L, np.float32(1.0)).astype(np.float32)
    t = ((g - lo[..., None]) / sc[..., None]).astype(np.float32)
    codes = np.rint(np.clip(t, np.float32(0.0), L)).astype(np.uint8).reshape(n, -1)
    return r, safe, codes, lo, sc


def gpu_group_compress(x: np.ndarray, R: np.ndarray, n_bits: int, group_size: int, P=None, rotate_fn=None):
    """compress_gpu (compress_kernel.py:100-189) on x [n, d]: y = clamp(x,
    +-65000) R^T in fp32 (rotate_fn(x, R), default the fp32 product in
    coordinate order, see the C restatement), the quantiser above, and the
    stored fields: radius fp16 (saturated at 65504), codes packed, lo and s
    fp16. With P ([m, d]): the QJL residual e = (y - (code s + lo)[:d] safe)
    R with the unrounded lo and s (fp32, two roundings each; the product back
    in fp32 by rotate_fn(., R, inverse)), signs (P e >= 0) in fp64 packed LSB
    first, and fp16 |e| (qjl_kernel.py:6-37). Returns a dict."""
    x = np.clip(np.asarray(x, np.float32), np.float32(-65000.0), np.float32(65000.0))
    n, d = x.shape
    if rotate_fn is None:
        def rotate_fn(v, M, inverse=False):
            M64 = np.asarray(M, np.float32).astype(np.float64)
            return (v.astype(np.float64) @ (M64 if inverse else M64.T)).astype(np.float32)
    y = rotate_fn(x, R)
    r, safe, codes, lo, sc = gpu_group_quantize(y, n_bits, group_size)
    out = {"radius": np.minimum(r, np.float32(65504.0)).astype(np.float16),
           "codes": gpu_group_pack(codes, n_bits), "mins": lo.astype(np.float16), "scales": sc.astype(np.float16),
           "codes_unpacked": codes, "y": y, "lo32": lo, "sc32": sc}
    if P is not None:
        ng = lo.shape[1]
        dq = (codes.reshape(n, ng, -1).astype(np.float32) * sc[..., None]).astype(np.float32) + lo[..., None]
        hat = dq.reshape(n, -1)[:, :d].astype(np.float32) * safe[:, None]
        e = rotate_fn((y - hat).astype(np.float32), R, inverse=True)
        proj = e.astype(np.float64) @ np.asarray(P, np.float64).T
        out["residual"] = e
        out["signs"] = bit_pack_lsb(proj >= 0)
        out["res_norms"] = np.sqrt((e.astype(np.float64) ** 2).sum(-1)).astype(np.float16)
    return out


def gpu_group_rotated(radius, codes_packed, mins, scales, d: int, n_bits: int) -> np.ndarray:
    """The rotated-space reconstruction (code s + lo)[:d] r of the stored
    fields, fp32 with two roundings for code s + lo and one for the product
    (decompress_kernel.py:34-43). [n, d] float32."""
    codes = gpu_group_unpack(codes_packed, n_bits).astype(np.float32)
    n = codes.shape[0]
    ng = np.asarray(mins).shape[-1]
    dq = (codes.reshape(n, ng, -1) * np.asarray(scales, np.float32)[..., None]).astype(np.float32) \
        + np.asarray(mins, np.float32)[..., None]
    return dq.reshape(n, -1)[:, :d].astype(np.float32) * np.asarray(radius, np.float32).reshape(n)[:, None]


def gpu_group_decompress(radius, codes_packed, mins, scales, R: np.ndarray, d: int, n_bits: int, group_size: int,
                         rotate_fn=None):
    """decompress_gpu (decompress_kernel.py:10-51): the rotated
    reconstruction above times R (rotate_fn(y, R, inverse=True), default the
    fp64 product), clamped to +-65504, fp16. Returns [n, d] float16."""
    y = gpu_group_rotated(radius, codes_packed, mins, scales, d, n_bits)
    if rotate_fn is None:
        out = y.astype(np.float64) @ np.asarray(R, np.float32).astype(np.float64)
    else:
        out = rotate_fn(y, R, inverse=True)
    return np.clip(out, -65504.0, 65504.0).astype(np.float16)


def group_attention(q: np.ndarray, K_hat: np.ndarray, V_hat: np.ndarray, scale: float | None = None,
                    signs=None, res_norms=None, P=None) -> np.ndarray:
    """compressed_attention_gpu's arithmetic after decompression
    (src/polarquant_kv_cuda/attention_kernel.py:62-113) and the CPU path's
    (python/polarquant_kv/attention.py:111-163), in float64: q [B, Hq, Sq, d]
    against K_hat / V_hat [B, Hkv, S, d] (the decompressed caches), GQA by
    repetition, s = q K_hat^T scale (+ scale (1/m) sum_i (2 sign_i - 1) (P q)_i
    with signs [B, Hkv, S, m/8], 0 where res_norms is 0: the guard of
    python/polarquant_kv/qjl.py:50-51), softmax over all S, w V_hat. S = 0
    gives zeros."""
    q = np.asarray(q, np.float64)
    B, Hq, Sq, d = q.shape
    Hkv, S = K_hat.shape[1], K_hat.shape[2]
    if S == 0:
        return np.zeros_like(q)
    scale = 1.0 / math.sqrt(d) if scale is None else float(scale)
    rep = Hq // Hkv
    K = np.repeat(np.asarray(K_hat, np.float64), rep, axis=1)
    V = np.repeat(np.asarray(V_hat, np.float64), rep, axis=1)
    s = np.einsum("bhqd,bhsd->bhqs", q, K) * scale
    if signs is not None and P is not None:
        m = P.shape[0]
        sv = 2.0 * bit_unpack_lsb(np.repeat(np.asarray(signs), rep, axis=1), m).astype(np.float64) - 1.0
        qp = q @ np.asarray(P, np.float64).T
        corr = np.einsum("bhqm,bhsm->bhqs", qp, sv) / m
        if res_norms is not None:
            live = np.repeat(np.asarray(res_norms, np.float64), rep, axis=1) > 1e-30
            corr = corr * live[:, :, None, :]
        s = s + corr * scale
    s = s - s.max(-1, keepdims=True)
    w = np.exp(s)
    w /= w.sum(-1, keepdims=True)
    return np.einsum("bhqs,bhsd->bhqd", w, V)


# ---------------------------------------------------------------------------
# GGML_TYPE_PQ4 and ggml's flash_attn_ext over it
# ---------------------------------------------------------------------------

def ggml_pq4_encode_rows(x: np.ndarray, d: int, R: np.ndarray, centroids: np.ndarray) -> np.ndarray:
    """PQ4 rows of x [n, k] float32 (k whole heads of d): per head the fp32
    FMA-chain rotation (the reference kernels' order, flash_turboquant.cu:
    132-137, as restated in pq_oracle.c), then quantize_rotated and
    pack_blocks (the radius tree, division, first-minimum scan, fp16 radius
    saturated at 65504). The table is the ggml init's (patch:978-983)."""
    from . import c_rotate_fma
    x = np.ascontiguousarray(x, np.float32)
    n, k = x.shape
    heads = x.reshape(-1, d)
    xr = c_rotate_fma(heads, R)
    r, idx = quantize_rotated(xr, centroids)
    return pack_blocks(r, idx, 4).reshape(n, -1)


def ggml_pq4_values(blocks: np.ndarray, d: int, R: np.ndarray, centroids: np.ndarray) -> np.ndarray:
    """The value of PQ4 heads [..., d/32 * 18] in float64: (r16 c[code]) R,
    the stored radius times the centroids rotated back (patch:508-544 applies
    x R to the attention output in the same space)."""
    b = np.asarray(blocks, np.uint8)
    lead = b.shape[:-1]
    rot = dequantize_rotated(b.reshape(-1, b.shape[-1]), d, centroids, 4).astype(np.float64)
    return (rot @ np.asarray(R, np.float64)).reshape(*lead, d)


def ggml_flash_attn_ext(q: np.ndarray, k: np.ndarray, v: np.ndarray, mask, scale: float) -> np.ndarray:
    """ggml_flash_attn_ext (ggml.h of ggml-org/llama.cpp, the upstream the
    reference's integration clones, integration/README.md:33; unpinned) in
    float64, with max_bias = logit_softcap = 0:
      q [ns][n_q][Hq][d], k / v [ns_k][n_kv][Hkv][d] (ns_k 1 or ns),
      mask None or [ns_m][n_q][n_kv] additive (ns_m 1 or ns);
      out[s][i][h] = sum_t w_t v[s][t][h // (Hq / Hkv)],
      w = softmax_t(scale q[s][i][h] . k[s][t][h // (Hq / Hkv)] + mask[s][i][t]);
    a row whose logits are all -inf is 0 (ggml's CPU kernel divides by a
    zero sum as 0). The reference's custom op computes the same attention
    without a mask (patch:1305-1362)."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    ns, n_q, Hq, d = q.shape
    Hkv = k.shape[2]
    G = Hq // Hkv
    out = np.zeros((ns, n_q, Hq, d))
    for s in range(ns):
        ks, vs = k[s if k.shape[0] > 1 else 0], v[s if v.shape[0] > 1 else 0]
        for i in range(n_q):
            m = None if mask is None else np.asarray(mask[s if mask.shape[0] > 1 else 0][i], np.float64)
            for h in range(Hq):
                logit = scale * (ks[:, h // G] @ q[s, i, h])
                if m is not None:
                    logit = logit + m
                mx = logit.max() if logit.size else -np.inf
                if not np.isfinite(mx):
                    continue
                w = np.exp(logit - mx)
                out[s, i, h] = (w @ vs[:, h // G]) / w.sum()
    return out


def synth_kv(B: int, H: int, S: int, d: int, seed: int, kind: str = "normal") -> np.ndarray:
    """fp16 K or V [B, H, S, d].

    normal:   i.i.d. N(0,1)
    token_ln: N(0,1) times a per-token LogNormal(0, 0.5) norm scale
    channel:  per-(head, channel) std ~ LogNormal(0,1), 1 % of channels x20
    """
    rng = np.random.Generator(np.random.PCG64(seed))
    x = rng.standard_normal((B, H, S, d), dtype=np.float32)
    if kind == "token_ln":
        x *= rng.lognormal(0.0, 0.5, size=(B, H, S, 1)).astype(np.float32)
    elif kind == "channel":
        std = rng.lognormal(0.0, 1.0, size=(1, H, 1, d)).astype(np.float32)
        n_out = max(1, int(round(0.01 * d)))
        for h in range(H):
            ch = rng.choice(d, size=n_out, replace=False)
            std[0, h, 0, ch] *= 20.0
        x *= std
    elif kind != "normal":
        raise ValueError(kind)
    return np.clip(x, -65504, 65504).astype(np.float16)
