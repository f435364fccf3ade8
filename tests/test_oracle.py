"""Pins of the CPU oracle: golden vectors written by the reference, closed
forms, special cases and brute force. Each check is chosen so that a plausible
slip (a transposed rotation, a dropped scale, a wrong nibble order, a reversed
tie rule, a different reduction order) fails it."""

import math

import numpy as np
import pytest

import oracle as oracle_pkg
from oracle import oracle as O

BOOKS = [(d, b) for d in (64, 128) for b in (2, 3, 4)]


# ---------------------------------------------------------------- codebook
@pytest.mark.parametrize("d,bits", BOOKS)
def test_codebook_matches_reference_golden(d, bits, golden_codebooks):
    c, b = O.lloyd_max_codebook(d, bits)
    gc, gb = golden_codebooks[f"d{d}_b{bits}"]
    assert np.array_equal(c, gc)
    assert np.array_equal(b, gb)


@pytest.mark.parametrize("d,bits", BOOKS)
def test_codebook_sorted_and_symmetric(d, bits):
    c, _ = O.lloyd_max_codebook(d, bits)
    assert np.all(np.diff(c) > 0)
    np.testing.assert_allclose(c, -c[::-1], atol=1e-6)


def test_codebook_gaussian_limit():
    # Max (1960) 16-level quantiser of N(0,1); the rotated coordinate has
    # variance 1/d and is close to Gaussian at d = 128.
    max16 = np.array([0.1284, 0.3881, 0.6568, 0.9424, 1.2562, 1.6180, 2.0690, 2.7326])
    c, _ = O.lloyd_max_codebook(128, 4)
    np.testing.assert_allclose(c[8:] * math.sqrt(128), max16, rtol=0.03)


# ---------------------------------------------------------------- rotation / JL
@pytest.mark.parametrize("d", [64, 128])
def test_rotation_matches_reference_golden(d, golden_R):
    R = O.rotation_matrix(d, 42)
    assert np.array_equal(R, golden_R[d])
    np.testing.assert_allclose(R.T @ R, np.eye(d), atol=1e-6)   # tests/test_rotation.py:15-23
    assert not np.allclose(R, O.rotation_matrix(d, 43))


def test_rotation_orientation():
    R = O.rotation_matrix(64, 42)
    v = np.random.default_rng(1).standard_normal((3, 64))
    np.testing.assert_allclose(O.rotate(v, R), (R @ v.T).T, atol=1e-12)
    np.testing.assert_allclose(O.inverse_rotate(O.rotate(v, R), R), v, atol=1e-12)


@pytest.mark.parametrize("key", [(64, 64, 43), (128, 128, 43), (64, 128, 42)])
def test_jl_matrix_matches_reference_golden(key, golden_P):
    m, d, s = key
    P = O.jl_matrix(m, d, s)
    assert np.array_equal(P, golden_P[key])
    assert abs(P.mean()) < 0.05 / math.sqrt(m)
    assert abs(P.var() * m - 1) < 0.05


# ---------------------------------------------------------------- quantiser
def _codebook(d, bits):
    return O.lloyd_max_codebook(d, bits)[0]


@pytest.mark.parametrize("d,bits", [(64, 4), (128, 4), (128, 2), (64, 2)])
def test_quantize_brute_force(d, bits):
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((300, d)) * rng.lognormal(0, 2, (300, 1))).astype(np.float32)
    c = _codebook(d, bits)
    r, idx = O.quantize_rotated(x, c)
    direction = (x / r[:, None]).astype(np.float32)
    dist = np.abs(direction[..., None] - c).astype(np.float32)
    assert np.array_equal(idx, dist.argmin(-1))            # first minimum wins
    np.testing.assert_allclose(r, np.linalg.norm(x.astype(np.float64), axis=1), rtol=1e-6)


U = 2.0 ** -23          # fp32 ulp of 1.0


def tree_probe(d):
    """x[0] = 1 and a run of slots at 2^-12 (squares delta = 2^-24, half an
    ulp of 1), the rest 0, so that the fp32 sum of squares depends on the
    order. Worked by hand through the 128-slot tree of
    csrc/flash_turboquant.cu:141-147 (slot t += slot t + s for s = 64, 32,
    ..., 1; d = 64 pads slots 64..127 with 0):

    d = 128, slots 64..127 set:
      s=64: slot 0 = 1 + delta -> 1 (tie, even);   slots 1..63 = delta
      s=32: slot 0 = 1 + delta -> 1;               slots 1..31 = U
      s=16: 1 + U;  s=8: 1 + 3U;  s=4: 1 + 7U;  s=2: 1 + 15U;  s=1: 1 + 31U
      r = RN(sqrt(1 + 31U)) = 1 + 15U   (exact sum 1 + 32U: r = 1 + 16U)
    d = 64, slots 1..12 set:
      s=64, 32, 16: nothing moves (the partner slots are 0)
      s=8: slot 0 = 1 + delta -> 1;  slots 1..4 = U;  slots 5..7 = delta
      s=4: slot 0 = 1 + U;  slots 1..3 = 1.5U
      s=2: slot 0 = 1 + 2.5U -> 1 + 2U (tie, even);  slot 1 = 3U
      s=1: 1 + 5U;  r = RN(sqrt(1 + 5U)) = 1 + 2U   (exact sum 1 + 6U: r = 1 + 3U)"""
    x = np.zeros((1, d), np.float32)
    x[0, 0] = 1.0
    if d == 128:
        x[0, 64:] = 2.0 ** -12
    else:
        x[0, 1:13] = 2.0 ** -12
    return x


def _other_orders(sq):
    """fp32 sums of squares in the orders a restatement could plausibly use."""
    out = {}
    acc = np.float32(0)
    for v in sq:
        acc = np.float32(acc + v)
    out["left_to_right"] = acc
    acc = np.float32(0)
    for v in sq[::-1]:
        acc = np.float32(acc + v)
    out["right_to_left"] = acc
    out["numpy_pairwise"] = np.sum(sq, dtype=np.float32)
    out["float64_rounded"] = np.float32(np.sum(sq.astype(np.float64)))
    b = np.concatenate([sq, np.zeros(128 - sq.size, np.float32)])
    while b.size > 1:                       # a tree over adjacent slot pairs
        b = (b[0::2] + b[1::2]).astype(np.float32)
    out["adjacent_pairs"] = b[0]
    return {k: np.sqrt(np.float32(v)) for k, v in out.items()}


@pytest.mark.parametrize("d,want_ulps", [(128, 15), (64, 2)])
def test_radius_tree_order_is_the_reference_one(d, want_ulps):
    x = tree_probe(d)
    r = O.radius_f32(x)[0]
    assert r == np.float32(1.0 + want_ulps * U)          # the hand-worked tree value
    for name, alt in _other_orders((x[0] * x[0]).astype(np.float32)).items():
        assert alt != r, f"the probe does not separate the tree from the {name} order"
    r_c, _ = oracle_pkg.c_quantize_rotated(x, _codebook(d, 4))
    assert r_c[0] == r


def test_identity_rotation_radius_is_the_norm():
    # integration patch test 2 (patch:2057-2061): R = I -> radius = |x|
    x = np.random.default_rng(3).standard_normal((50, 128)).astype(np.float32)
    xr, r, _ = O.encode(x, np.eye(128), _codebook(128, 4))
    np.testing.assert_array_equal(xr, x)
    np.testing.assert_allclose(r, np.linalg.norm(x.astype(np.float64), axis=1), rtol=1e-6)


def test_zero_vector():
    c = _codebook(128, 4)
    r, idx = O.quantize_rotated(np.zeros((1, 128), np.float32), c)
    assert r[0] == 0.0
    assert np.all(idx == np.argmin(np.abs(c)))


def test_quantiser_is_idempotent():
    # A vector built from the centroids of a quantised direction (norm ~1)
    # quantises back to the same codes.
    rng = np.random.default_rng(5)
    for d, bits in ((128, 4), (64, 4), (128, 2)):
        c = _codebook(d, bits)
        _, want = O.quantize_rotated(rng.standard_normal((64, d)).astype(np.float32), c)
        _, idx = O.quantize_rotated(c[want] * np.float32(3.0), c)
        assert np.array_equal(idx, want)


def test_c_and_numpy_restatements_agree():
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((2000, 128)) * rng.lognormal(0, 3, (2000, 1))).astype(np.float32)
    x[0] = 0
    x[1] = 1e-30
    for bits in (2, 4):
        c = _codebook(128, bits)
        r1, i1 = O.quantize_rotated(x, c)
        r2, i2 = oracle_pkg.c_quantize_rotated(x, c)
        assert np.array_equal(r1.view(np.uint32), r2.view(np.uint32))
        assert np.array_equal(i1, i2)
        assert np.array_equal(O.pack_blocks(r1, i1, bits), oracle_pkg.c_pack_blocks(r2, i2, bits))


def test_c_fma_rotation_close_to_float64():
    x = np.random.default_rng(2).standard_normal((20, 128)).astype(np.float32)
    R = O.rotation_matrix(128, 42).astype(np.float32)
    y = oracle_pkg.c_rotate_fma(x, R)
    np.testing.assert_allclose(y, x.astype(np.float64) @ R.astype(np.float64).T, atol=2e-6)
    np.testing.assert_allclose(oracle_pkg.c_rotate_fma(y, R, inverse=True), x, atol=5e-6)


# ---------------------------------------------------------------- packing
def test_nibble_order_kat():
    # scripts/debug_kernel2.py:58-63: bytes A5 83 27 1C hold 5,10,3,8,7,2,12,1
    codes = np.array([5, 10, 3, 8, 7, 2, 12, 1], np.uint8)
    packed = np.array([0xA5, 0x83, 0x27, 0x1C], np.uint8)
    assert np.array_equal(O.pack_codes(codes, 4), packed)
    assert np.array_equal(O.unpack_codes(packed, 4), codes)


def test_crumb_order():
    # compress_kernel.py:43-50: v0 | v1 << 2 | v2 << 4 | v3 << 6
    codes = np.array([1, 2, 3, 0, 3, 3, 0, 1], np.uint8)
    packed = O.pack_codes(codes, 2)
    assert list(packed) == [1 | 2 << 2 | 3 << 4, 3 | 3 << 2 | 0 << 4 | 1 << 6]
    assert np.array_equal(O.unpack_codes(packed, 2), codes)


def test_stored_radius_saturates_at_fp16_max():
    # compress_kernel.py:178 stores radius.clamp(-65504, 65504).half(): a norm
    # past the fp16 range is kept as 65504 (0x7BFF), never inf; NaN stays NaN.
    r = np.array([65504.0, 65519.0, 65520.0, 1.1e5, np.inf, np.nan, 1.0], np.float32)
    idx = np.zeros((r.size, 32), np.uint8)
    for bits in (4, 2):
        for blk in (O.pack_blocks(r, idx, bits), oracle_pkg.c_pack_blocks(r, idx, bits)):
            r16 = blk[:, 0].astype(np.uint16) | (blk[:, 1].astype(np.uint16) << 8)
            assert list(r16[:5]) == [0x7BFF] * 5
            assert (r16[5] & 0x7C00) == 0x7C00 and (r16[5] & 0x3FF) != 0
            assert r16[6] == 0x3C00


@pytest.mark.parametrize("d,bits", [(128, 4), (64, 4), (128, 2), (64, 2)])
def test_block_layout_round_trip(d, bits):
    rng = np.random.default_rng(9)
    idx = rng.integers(0, 1 << bits, size=(10, d)).astype(np.uint8)
    r = rng.lognormal(0, 2, 10).astype(np.float32)
    blk = O.pack_blocks(r, idx, bits)
    assert blk.shape == (10, O.vector_bytes(d, bits))
    assert O.vector_bytes(128, 4) == 72 and O.vector_bytes(64, 4) == 36 and O.vector_bytes(128, 2) == 40
    r16, idx2 = O.unpack_blocks(blk, d, bits)
    assert np.array_equal(idx2, idx)
    assert np.array_equal(r16, r.astype(np.float16))
    # every block repeats the radius
    nb = d // 32
    bb = O.block_bytes(bits)
    for b in range(nb):
        assert np.array_equal(blk[:, b * bb:b * bb + 2], blk[:, 0:2])


# ---------------------------------------------------------------- attention
def _random_cache(rng, B, H, S, d, bits=4, kind="normal"):
    c = _codebook(d, bits)
    x = O.synth_kv(B, H, S, d, int(rng.integers(1 << 30)), kind).astype(np.float32)
    R = O.rotation_matrix(d, 42)
    xr = O.rotate(x.reshape(-1, d), R).astype(np.float32)
    r, idx = O.quantize_rotated(xr, c)
    return O.pack_blocks(r, idx, bits).reshape(B, H, S, -1), c, R


def test_decode_equals_textbook_attention_on_dequantised_cache():
    rng = np.random.default_rng(0)
    B, Hq, Hkv, S, d = 2, 4, 2, 37, 64
    kb, c, R = _random_cache(rng, B, Hkv, S, d)
    vb, _, _ = _random_cache(rng, B, Hkv, S, d)
    q = rng.standard_normal((B, Hq, d))
    out = O.decode_attention(q, kb, vb, R, c, c)
    K = O.inverse_rotate(O.dequantize_rotated(kb, d, c), R)     # original space
    V = O.inverse_rotate(O.dequantize_rotated(vb, d, c), R)
    g = Hq // Hkv
    for h in range(Hq):
        ref = O.sdpa(q[:, h:h + 1], K[:, h // g], V[:, h // g])[:, 0]
        np.testing.assert_allclose(out[:, h], ref, atol=1e-10)


def test_decode_gqa_equals_repeated_heads():
    rng = np.random.default_rng(1)
    kb, c, R = _random_cache(rng, 1, 2, 20, 128)
    vb, _, _ = _random_cache(rng, 1, 2, 20, 128)
    q = rng.standard_normal((1, 8, 128))
    a = O.decode_attention(q, kb, vb, R, c, c)
    b = O.decode_attention(q, np.repeat(kb, 4, axis=1), np.repeat(vb, 4, axis=1), R, c, c)
    np.testing.assert_allclose(a, b, atol=1e-12)


def test_decode_empty_sequence_gives_zeros():
    kb = np.zeros((1, 1, 0, 72), np.uint8)
    out = O.decode_attention(np.ones((1, 2, 128)), kb, kb, np.eye(128), _codebook(128, 4), _codebook(128, 4))
    assert np.all(out == 0) and out.shape == (1, 2, 128)


def test_prefill_matches_masked_textbook_attention():
    rng = np.random.default_rng(4)
    B, Hq, Hkv, S, d, Sq = 1, 2, 1, 24, 64, 6
    kb, c, R = _random_cache(rng, B, Hkv, S, d)
    vb, _, _ = _random_cache(rng, B, Hkv, S, d)
    q = rng.standard_normal((B, Hq, Sq, d))
    q0 = S - Sq
    out = O.prefill_attention(q, kb, vb, R, c, c, q_start=q0, causal=True)
    K = O.inverse_rotate(O.dequantize_rotated(kb, d, c), R)[:, 0]
    V = O.inverse_rotate(O.dequantize_rotated(vb, d, c), R)[:, 0]
    s = q @ np.swapaxes(K, -1, -2)[:, None] / math.sqrt(d)          # [B, Hq, Sq, S]
    mask = np.arange(S)[None, :] <= (q0 + np.arange(Sq))[:, None]
    s = np.where(mask, s, -np.inf)
    w = np.exp(s - s.max(-1, keepdims=True))
    w /= w.sum(-1, keepdims=True)
    np.testing.assert_allclose(out, w @ V[:, None], atol=1e-10)


# ---------------------------------------------------------------- QJL
def test_qjl_closed_form_and_rotated_identity():
    rng = np.random.default_rng(6)
    d = 64
    R = O.rotation_matrix(d, 42)
    P = O.jl_matrix(d, d, 43)
    c = _codebook(d, 4)
    x = rng.standard_normal((10, d)).astype(np.float32)
    xr = O.rotate(x, R).astype(np.float32)
    r, idx = O.quantize_rotated(xr, c)
    signs, norms = O.qjl_signs_rotated(xr, r, idx, c, P @ R.T)
    e_orig = O.inverse_rotate(xr.astype(np.float64) - r[:, None] * c[idx].astype(np.float64), R)
    assert np.array_equal(signs, O.bit_pack_lsb(e_orig @ P.T >= 0))
    np.testing.assert_allclose(norms, np.linalg.norm(e_orig, axis=1), rtol=1e-9)
    # correction = (1/m) sum_i (2 s_i - 1) (P q)_i, written as an explicit loop
    q = rng.standard_normal(d)
    corr = O.qjl_correction(q[None], signs, P)[0]
    bits = O.bit_unpack_lsb(signs, d)
    for t in range(10):
        want = sum((1.0 if bits[t, i] else -1.0) * float(P[i] @ q) for i in range(d)) / d
        assert abs(corr[t] - want) < 1e-12


# Code vectors whose centroids c[idx] have an fp32 tree radius of exactly 1.0
# (found by a meet-in-the-middle search over the 4-bit Lloyd-Max codebook; the
# property is checked below), so x_rot = 2 c[idx] encodes losslessly: r = 2,
# dir = c[idx], residual 0.
LOSSLESS_IDX = {
    64: [1, 8, 3, 7, 11, 10, 11, 12, 10, 10, 1, 13, 2, 8, 8, 10, 7, 5, 4, 9, 10, 8, 8, 3, 9, 3, 6, 5, 2, 10, 13,
         10, 10, 4, 10, 13, 10, 4, 8, 6, 6, 14, 5, 5, 10, 4, 3, 1, 3, 5, 5, 9, 8, 13, 10, 6, 8, 14, 8, 11, 13, 5,
         11, 9],
    128: [6, 9, 7, 5, 3, 13, 8, 9, 0, 4, 10, 5, 5, 8, 4, 5, 4, 9, 5, 12, 2, 9, 10, 2, 7, 4, 4, 12, 9, 4, 3, 10, 5,
          9, 11, 8, 6, 3, 9, 3, 0, 7, 9, 0, 9, 10, 10, 13, 3, 4, 6, 5, 2, 8, 3, 8, 2, 11, 7, 2, 4, 3, 7, 12, 10, 8,
          12, 4, 5, 10, 13, 6, 5, 8, 6, 8, 11, 3, 5, 8, 11, 7, 3, 7, 7, 2, 10, 0, 10, 4, 1, 11, 6, 3, 7, 5, 3, 11,
          5, 9, 9, 6, 6, 2, 5, 6, 11, 12, 11, 5, 7, 8, 12, 6, 11, 14, 1, 8, 11, 4, 7, 4, 8, 7, 6, 8, 11, 9],
}


def lossless_key(d, scale=2.0):
    return (np.float32(scale) * _codebook(d, 4)[np.array(LOSSLESS_IDX[d])]).astype(np.float32)


@pytest.mark.parametrize("d", [64, 128])
def test_lossless_key_has_zero_residual(d):
    c = _codebook(d, 4)
    x = lossless_key(d)[None]
    r, idx = O.quantize_rotated(x, c)
    assert r[0] == np.float32(2.0)
    assert np.array_equal(idx[0], LOSSLESS_IDX[d])
    signs, enorm = O.qjl_signs_rotated(x, r, idx, c, O.jl_matrix(d, d, 43))
    assert enorm[0] == 0.0 and np.all(signs == 0xFF)      # P 0 = 0 >= 0: every sign 1


def qjl_rule_cache(d=64, S=6, seed=12, key_scale=1.0):
    """One (batch, kv-head) stream whose key 0 is the zero vector and key 1 is
    lossless (residual 0); the rest are random. Signs as the encoder writes
    them: P 0 = 0 >= 0 gives all ones for keys 0 and 1.
    Returns (k_blocks, v_blocks, signs, P, R, c, x_rot)."""
    rng = np.random.default_rng(seed)
    c = _codebook(d, 4)
    R = O.rotation_matrix(d, 42)
    P = O.jl_matrix(d, d, 43)
    xr = (key_scale * rng.standard_normal((S, d))).astype(np.float32)
    xr[0] = 0.0
    xr[1] = lossless_key(d)
    r, idx = O.quantize_rotated(xr, c)
    signs, enorm = O.qjl_signs_rotated(xr, r, idx, c, P @ R.T)
    assert enorm[0] == 0.0 and enorm[1] == 0.0 and np.all(enorm[2:] > 0)
    assert np.all(signs[:2] == 0xFF)
    kb = O.pack_blocks(r, idx, 4)
    vr = rng.standard_normal((S, d)).astype(np.float32)
    rv, iv = O.quantize_rotated(vr, c)
    vb = O.pack_blocks(rv, iv, 4)
    return kb[None, None], vb[None, None], signs[None, None], P, R, c, xr


def test_qjl_zero_residual_keys_get_no_correction():
    """The rule (reference AC-3.5, tests/test_qjl.py:139-154, guard at
    python/polarquant_kv/qjl.py:50-51): a key whose residual is zero adds no
    correction. Key 0 is the zero vector and key 1 is lossless (rotated-space
    residual 0); both store an all-ones sketch (P 0 = 0 >= 0), and a block
    cache keeps no residual norm, so the all-ones sketch marks them. Every
    other key adds (1/m) sum_i (2 s_i - 1) (P q)_i
    (src/polarquant_kv_cuda/attention_kernel.py:95-107). Scores assembled by
    hand here; a kernel that dropped the guard (both corrected) or guarded on
    the radius only (lossless key corrected) fails."""
    d, S, G = 64, 6, 2
    kb, vb, signs, P, R, c, xr = qjl_rule_cache(d, S)
    assert np.array_equal(O.qjl_zero_residual(signs[0, 0], d), [True, True] + [False] * (S - 2))
    q = np.random.default_rng(3).standard_normal((1, G, d))
    got = O.decode_attention(q, kb, vb, R, c, c, qjl_signs=signs, P=P)
    r16, idx = O.unpack_blocks(kb[0, 0], d, 4)
    K = r16.astype(np.float64)[:, None] * c[idx].astype(np.float64)
    Vr = O.dequantize_rotated(vb[0, 0], d, c)
    bits = O.bit_unpack_lsb(signs[0, 0], d).astype(np.float64) * 2 - 1
    scale = 1 / math.sqrt(d)
    for g in range(G):
        qr = R @ q[0, g]
        pq = P @ q[0, g]
        s = np.array([qr @ K[t] + (0.0 if t < 2 else bits[t] @ pq / d) for t in range(S)]) * scale
        assert s[0] == 0.0
        assert abs(s[1] - scale * (qr @ K[1])) < 1e-12
        w = np.exp(s - s.max())
        w /= w.sum()
        np.testing.assert_allclose(got[0, g], (w @ Vr) @ R, atol=1e-12)
    # the other rules give different scores on this cache
    pq0 = P @ q[0, 0]
    assert abs(bits[0] @ pq0 / d) > 1e-3 and abs(bits[1] @ pq0 / d) > 1e-3


def test_qjl_zero_residual_needs_every_sign():
    """One clear bit anywhere in the sketch (any byte, any bit) means a
    non-zero residual: the mask is an AND over all m signs."""
    m = 64
    full = np.full((m + 1, m // 8), 0xFF, np.uint8)
    for i in range(m):
        full[i + 1, i // 8] &= ~np.uint8(1 << (i % 8))
    z = O.qjl_zero_residual(full, m)
    assert z[0] and not z[1:].any()


def test_bit_pack_lsb_round_trip():
    s = np.random.default_rng(0).random((3, 13)) > 0.5
    p = O.bit_pack_lsb(s)
    assert p.shape == (3, 2)
    assert np.array_equal(O.bit_unpack_lsb(p, 13), s)
    assert O.bit_pack_lsb(np.array([True] + [False] * 7))[0] == 1     # bit 0 is the first sign


def test_soa_attention_equals_block_attention_on_fp16_exact_radii():
    """decode_attention_soa (fp32 radii as given) against the pinned block
    decode with an identity rotation: radii that fp16 holds exactly give the
    same scores, so the two agree to rounding; radii that fp16 rounds give a
    measurable difference (the reason the SoA path keeps fp32 radii)."""
    rng = np.random.default_rng(21)
    Hq, Hkv, S, d = 6, 2, 50, 64
    c = _codebook(d, 4)
    idx_k = rng.integers(0, 16, (Hkv * S, d)).astype(np.uint8)
    idx_v = rng.integers(0, 16, (Hkv * S, d)).astype(np.uint8)
    rk = rng.lognormal(2, 1, Hkv * S).astype(np.float16).astype(np.float32)     # fp16-exact
    rv = rng.lognormal(2, 1, Hkv * S).astype(np.float16).astype(np.float32)
    q = rng.standard_normal((Hq, d))
    pk, pv = O.pack_codes(idx_k, 4), O.pack_codes(idx_v, 4)
    got = O.decode_attention_soa(q, pk, rk, pv, rv, c, Hkv, 1 / math.sqrt(d))
    kb = O.pack_blocks(rk, idx_k, 4).reshape(1, Hkv, S, -1)
    vb = O.pack_blocks(rv, idx_v, 4).reshape(1, Hkv, S, -1)
    want = O.decode_attention(q[None], kb, vb, np.eye(d), c, c)[0]
    np.testing.assert_allclose(got, want, atol=1e-10)
    rk2 = rk * np.float32(1 + 2 ** -13)                       # not fp16 numbers any more
    moved = O.decode_attention_soa(q, pk, rk2, pv, rv * np.float32(1 + 2 ** -13), c, Hkv, 1 / math.sqrt(d))
    assert np.abs(moved - want).max() > 1e-6


def test_ggml_codebook_fixture():
    import json
    import os
    from conftest import GOLDEN
    books = json.load(open(os.path.join(GOLDEN, "ggml_codebooks.json")))["codebooks"]
    for bits, vals in books.items():
        assert len(vals) == 1 << int(bits) and np.all(np.diff(vals) > 0)
    # the reference's 4-bit table is not the Lloyd-Max table (asymmetric,
    # narrower): ggml callers get codes of their own codebook
    assert not np.allclose(books["4"], _codebook(128, 4), atol=1e-3)
