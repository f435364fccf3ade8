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


def test_radius_tree_order_is_the_reference_one():
    # Values whose fp32 sum depends on association order: the 128-slot tree
    # (pairs t, t+64 first) must be used, not a left-to-right sum.
    x = np.zeros((1, 128), np.float32)
    x[0, 0], x[0, 64], x[0, 1] = 1.0, 2.0 ** -12, 2.0 ** -12
    r2_tree = O.radius_f32(x)[0] ** 2
    seq = np.float32(0)
    for v in (x[0] * x[0]):
        seq = np.float32(seq + v)
    pairs = np.float32(np.float32(x[0, 0] ** 2 + x[0, 64] ** 2) + np.float32(x[0, 1] ** 2))
    assert np.float32(np.sqrt(pairs)) == O.radius_f32(x)[0]
    assert r2_tree > 0 and seq > 0


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


def test_bit_pack_lsb_round_trip():
    s = np.random.default_rng(0).random((3, 13)) > 0.5
    p = O.bit_pack_lsb(s)
    assert p.shape == (3, 2)
    assert np.array_equal(O.bit_unpack_lsb(p, 13), s)
    assert O.bit_pack_lsb(np.array([True] + [False] * 7))[0] == 1     # bit 0 is the first sign
