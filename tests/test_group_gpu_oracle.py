"""Pins of the oracle's restatement of the reference's GPU group format
(src/polarquant_kv_cuda/compress_kernel.py:100-189, decompress_kernel.py:10-51,
attention_kernel.py:62-113): hand-worked codes (padding inside the min / max,
flat groups, the zero vector), the packing orders, the residual of a
hand-worked vector, the reference tests' round-trip cosine thresholds
(tests/cuda/test_compress_decompress.py:66-80), and the attention against
torch's float64 SDPA and a hand-applied zero-residual guard."""

import math

import numpy as np
import torch

from oracle import oracle as O


def _eye(d):
    return np.eye(d)


def test_hand_worked_codes_with_padding_inside_the_group():
    # d = 6, group_size = 4: the last group is [0.6, 0.8, 0, 0] after the
    # zero padding, so its minimum is 0 (not 0.6) and its scale 0.8 / 15
    y = np.array([[0, 0, 0, 0, 0.6, 0.8]], np.float32)
    r, safe, codes, lo, sc = O.gpu_group_quantize(y, 4, 4)
    assert r[0] == np.float32(1.0)
    assert lo[0, 0] == 0 and sc[0, 0] == 1.0                  # flat first group: scale 1, codes 0
    assert lo[0, 1] == 0 and sc[0, 1] == np.float32(np.float32(0.8) / np.float32(15))
    # 0.6 / (0.8 / 15) = 11.25 -> 11, 0.8 -> 15, the padding -> 0
    assert codes[0].tolist() == [0, 0, 0, 0, 11, 15, 0, 0]


def test_hand_worked_codes_three_four():
    y = np.array([[3, 4, 0, 0, 0, 0, 0, 0]], np.float32)
    r, safe, codes, lo, sc = O.gpu_group_quantize(y, 4, 8)
    assert r[0] == 5 and safe[0] == 5
    assert codes[0].tolist() == [11, 15, 0, 0, 0, 0, 0, 0]
    # 2 bits: scale 0.8 / 3; 0.6 / s = 2.25 -> 2, 0.8 -> 3
    assert O.gpu_group_quantize(y, 2, 8)[2][0].tolist() == [2, 3, 0, 0, 0, 0, 0, 0]
    # 8 bits: 0.6 / (0.8 / 255) = 191.25 -> 191
    assert O.gpu_group_quantize(y, 8, 8)[2][0].tolist()[:2] == [191, 255]


def test_zero_vector():
    y = np.zeros((1, 8), np.float32)
    r, safe, codes, lo, sc = O.gpu_group_quantize(y, 4, 4)
    assert r[0] == 0 and safe[0] == np.float32(1e-30)
    assert not codes.any() and not lo.any() and (sc == 1).all()
    out = O.gpu_group_compress(y, _eye(8), 4, 4, P=O.jl_matrix(16, 8, 1))
    assert out["radius"][0] == 0 and not out["residual"].any()
    assert (out["signs"] == 0xFF).all() and out["res_norms"][0] == 0      # P 0 = 0 >= 0


def test_packing_orders():
    codes = np.array([[1, 2, 3, 4, 15, 0, 7, 8]], np.uint8)
    assert O.gpu_group_pack(codes, 4).tolist() == [[0x21, 0x43, 0x0F, 0x87]]     # high << 4 | low
    c2 = np.array([[1, 2, 3, 0, 3, 3, 3, 3]], np.uint8)
    assert O.gpu_group_pack(c2, 2).tolist() == [[0x39, 0xFF]]                   # v0 | v1<<2 | v2<<4 | v3<<6
    c8 = np.array([[200, 7]], np.uint8)
    assert O.gpu_group_pack(c8, 3).tolist() == [[200, 7]]                       # other widths: bytes
    for bits, c in ((4, codes), (2, c2)):
        assert np.array_equal(O.gpu_group_unpack(O.gpu_group_pack(c, bits), bits), c)


def test_hand_worked_residual_and_reconstruction():
    # R = I, y = (3, 4, 0 ...): codes 11, 15 with s = 0.8 / 15 and r = 5, so
    # the reconstruction is (11 s, 15 s) 5 and the residual y minus it
    y = np.array([[3, 4, 0, 0, 0, 0, 0, 0]], np.float32)
    out = O.gpu_group_compress(y, _eye(8), 4, 8, P=O.jl_matrix(32, 8, 2))
    s = np.float32(0.8) / np.float32(15)
    want = np.array([3 - 11 * float(s) * 5, 4 - 15 * float(s) * 5] + [0] * 6)
    np.testing.assert_allclose(out["residual"][0], want, atol=1e-6)
    assert abs(out["residual"][0, 0] - 1 / 15) < 1e-5
    xh = O.gpu_group_decompress(out["radius"], out["codes"], out["mins"], out["scales"], _eye(8), 8, 4, 8)
    # from the fp16 fields: s16 = fp16(0.8/15), r16 = 5
    s16 = float(np.float16(s))
    np.testing.assert_allclose(xh[0, :2].astype(np.float64), [11 * s16 * 5, 15 * s16 * 5], rtol=1e-3)


def test_round_trip_cosine_thresholds_of_the_reference_tests():
    # tests/cuda/test_compress_decompress.py:66-80: average per-vector
    # cosine of decompress(compress(kv)) against kv, 16 fp16 N(0,1) vectors
    d = 128
    R = O.rotation_matrix(d, 42)
    x = np.random.default_rng(42).standard_normal((16, d)).astype(np.float16).astype(np.float32)
    for bits, thr in ((4, 0.99), (3, 0.96), (2, 0.88)):
        o = O.gpu_group_compress(x, R, bits, 32)
        xh = O.gpu_group_decompress(o["radius"], o["codes"], o["mins"], o["scales"], R, d, bits, 32)
        xh = xh.astype(np.float64)
        cos = (x * xh).sum(1) / np.linalg.norm(x, axis=1) / np.linalg.norm(xh, axis=1)
        assert cos.mean() >= thr, (bits, cos.mean())


def test_group_attention_is_sdpa_on_the_decompressed_caches():
    rng = np.random.default_rng(3)
    B, Hq, Hkv, Sq, S, d = 2, 6, 2, 3, 40, 64
    q = rng.standard_normal((B, Hq, Sq, d))
    K = rng.standard_normal((B, Hkv, S, d))
    V = rng.standard_normal((B, Hkv, S, d))
    got = O.group_attention(q, K, V)
    rep = Hq // Hkv
    want = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q), torch.from_numpy(np.repeat(K, rep, 1)).contiguous(),
        torch.from_numpy(np.repeat(V, rep, 1)).contiguous()).numpy()
    np.testing.assert_allclose(got, want, atol=1e-12)
    assert not O.group_attention(q, K[:, :, :0], V[:, :, :0]).any()


def test_group_attention_zero_residual_guard_by_hand():
    rng = np.random.default_rng(4)
    d, S, m = 32, 5, 32
    q = rng.standard_normal((1, 1, 1, d))
    K = rng.standard_normal((1, 1, S, d))
    V = rng.standard_normal((1, 1, S, d))
    P = O.jl_matrix(m, d, 7)
    bits = rng.random((S, m)) > 0.5
    signs = O.bit_pack_lsb(bits)[None, None]
    norms = np.array([0.0, 1.0, 2.0, 0.0, 3.0])[None, None]
    got = O.group_attention(q, K, V, signs=signs, res_norms=norms, P=P)[0, 0, 0]
    pq = P @ q[0, 0, 0]
    s = np.array([q[0, 0, 0] @ K[0, 0, t] + (0.0 if norms[0, 0, t] == 0 else
                                            (2.0 * bits[t] - 1) @ pq / m) for t in range(S)]) / math.sqrt(d)
    w = np.exp(s - s.max())
    np.testing.assert_allclose(got, (w / w.sum()) @ V[0, 0], atol=1e-12)
    # without the guard the zero-residual keys would be corrected
    unguarded = O.group_attention(q, K, V, signs=signs, res_norms=None, P=P)[0, 0, 0]
    assert np.abs(unguarded - got).max() > 1e-3
