"""The group (min / scale) oracle pinned on the CPU: hand-worked codes, the
zero vector, padding, and the reference tests' quality thresholds
(tests/test_quantizer.py:66-110 of the reference)."""

import numpy as np
import pytest

from oracle import oracle as O


def test_round_half_to_even_and_flat_groups():
    # scale 0.75 / 3 = 0.25 exactly: 0.375 -> 1.5 -> 2, 0.625 -> 2.5 -> 2
    codes, lo, sc = O.group_quantize_direction(np.array([0, 0.75, 0.375, 0.625], np.float32), 2, 4)
    assert codes.tolist() == [0, 3, 2, 2] and lo[0] == 0 and sc[0] == 0.25
    # a flat group: scale 1, codes 0
    codes, lo, sc = O.group_quantize_direction(np.array([0.5, 0.5, 0.1, 0.3], np.float32), 4, 2)
    assert codes.tolist() == [0, 0, 0, 15] and sc[0] == 1.0 and lo[0] == 0.5
    # padding: d = 5, group 4 -> 8 codes, the last group's pad zeros count
    codes, lo, sc = O.group_quantize_direction(np.array([1, 2, 3, 4, -0.5], np.float32), 2, 4)
    assert codes.shape == (8,) and lo[1] == -0.5 and codes[5:].tolist() == [3, 3, 3]


def test_compress_identity_rotation_hand_case():
    # R = I: y = v, r = 5, u = (0.6, 0, 0, 0.8)
    r, codes, lo, sc = O.group_compress(np.array([3, 0, 0, 4], np.float32), np.eye(4), 2, 2)
    assert r == np.float32(5.0)
    assert codes.tolist() == [3, 0, 0, 3]
    assert np.array_equal(lo, np.float32([0, 0]))
    out = O.group_decompress(r, codes, lo, sc, np.eye(4), 4, 2)
    assert np.allclose(out, [3, 0, 0, 4], atol=1e-6)


def test_zero_vector():
    R = O.rotation_matrix(64, 42)
    r, codes, lo, sc = O.group_compress(np.zeros(64, np.float32), R, 4, 32)
    assert r == 0 and not codes.any() and not lo.any() and (sc == 1).all()
    assert not O.group_decompress(r, codes, lo, sc, R, 64, 32).any()


@pytest.mark.parametrize("n_bits,threshold", [(4, 0.99), (3, 0.98), (2, 0.92), (6, 0.995), (8, 0.999)])
def test_reference_cosine_thresholds(n_bits, threshold):
    d = 128
    R = O.rotation_matrix(d, 42)
    sims = []
    for i in range(20):
        v = np.random.Generator(np.random.PCG64(42 + i)).standard_normal(d).astype(np.float32)
        r, c, lo, sc = O.group_compress(v, R, n_bits, 32)
        w = O.group_decompress(r, c, lo, sc, R, d, 32)
        sims.append(float(v @ w / (np.linalg.norm(v) * np.linalg.norm(w))))
    assert np.mean(sims) >= threshold


def test_padding_reference_case():
    d = 100
    R = O.rotation_matrix(d, 42)
    v = np.random.Generator(np.random.PCG64(42)).standard_normal(d).astype(np.float32)
    r, c, lo, sc = O.group_compress(v, R, 4, 32)
    w = O.group_decompress(r, c, lo, sc, R, d, 32)
    assert c.shape == (128,) and w.shape == (d,)
    assert float(v @ w / (np.linalg.norm(v) * np.linalg.norm(w))) >= 0.98
