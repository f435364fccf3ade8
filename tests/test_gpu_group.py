"""The group (min / scale) quantizer API (polarquant_kv.quantizer.compress /
decompress / compress_batch / decompress_batch) on the GPU against the
oracle restatement of the reference's CPU quantizer, and the reference
tests' own checks (tests/test_quantizer.py, tests/test_batch.py)."""

import numpy as np
import pytest

from oracle import oracle as O
from polarquant_kv import quantizer, rotation
from polarquant_kv.types import CompressedKV
from polarquant_kv.utils import cosine_similarity

pytestmark = pytest.mark.gpu


def _ulps(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return np.abs(a.view(np.int32).astype(np.int64) - b.view(np.int32).astype(np.int64))


@pytest.mark.parametrize("d,bits,gs", [(128, 4, 32), (128, 2, 16), (100, 3, 32), (64, 8, 7), (32, 6, 32),
                                       (256, 4, 64), (128, 4, 1)])
def test_group_arrays_match_the_oracle(d, bits, gs):
    print(f"group d={d} bits={bits} gs={gs}", flush=True)
    rng = np.random.default_rng(d * bits + gs)
    n = 1500
    x = (rng.standard_normal((n, d)) * rng.lognormal(0, 1, (n, 1))).astype(np.float32)
    x[0] = 0.0
    x[1, :] = 0.0
    x[1, 3] = 2.0
    R = rotation.generate_rotation_matrix(d, seed=42)
    r, codes, lo, sc = quantizer.group_compress_arrays(x, R, bits, gs)
    ref = [O.group_compress(x[i], R, bits, gs) for i in range(n)]
    r_ref = np.array([t[0] for t in ref], np.float32)
    assert _ulps(r, r_ref).max() <= 2                      # fp64 vs numpy fp32 norm
    assert r[0] == 0 and not codes[0].any() and (sc[0] == 1).all()
    same = np.array([np.array_equal(codes[i], ref[i][1]) for i in range(n)])
    assert same.mean() > 0.995, same.mean()
    # a differing code is one step off, where the oracle's pre-round value
    # is within rounding of a half (the radius differs by an ulp)
    for i in np.flatnonzero(~same)[:50]:
        assert np.abs(codes[i].astype(int) - ref[i][1].astype(int)).max() == 1
    ok = np.flatnonzero(same & (r == r_ref))
    assert np.array_equal(np.stack([lo[i] for i in ok]), np.stack([ref[i][2] for i in ok]))
    assert np.array_equal(np.stack([sc[i] for i in ok]), np.stack([ref[i][3] for i in ok]))
    # decompression of the GPU's own codes against the oracle's
    out = quantizer.group_decompress_arrays(r, codes, lo, sc, R, d, gs)
    want = np.stack([O.group_decompress(r[i], codes[i], lo[i], sc[i], R, d, gs) for i in range(n)])
    err = np.abs(out.astype(np.float64) - want) / (np.abs(want).max(axis=1, keepdims=True) + 1e-30)
    assert err.max() <= 2.0 ** -22, err.max()
    assert not out[0].any()


def test_fp16_input_is_rotated_as_fp32():
    d = 128
    R = rotation.generate_rotation_matrix(d, seed=42)
    v = np.random.default_rng(0).standard_normal(d).astype(np.float16)
    c16 = quantizer.compress(v, R)
    c32 = quantizer.compress(v.astype(np.float32), R)
    assert c16.radius == c32.radius and np.array_equal(c16.quantized_direction, c32.quantized_direction)
    out = quantizer.decompress(c16, R)
    assert out.dtype == np.float32 and out.shape == (d,)


@pytest.mark.parametrize("n_bits,threshold", [(4, 0.99), (3, 0.98), (2, 0.92), (6, 0.995), (8, 0.999)])
def test_reference_cosine_thresholds(n_bits, threshold):
    d = 128
    R = rotation.generate_rotation_matrix(d, seed=42)
    sims = []
    for i in range(20):
        v = np.random.Generator(np.random.PCG64(42 + i)).standard_normal(d).astype(np.float32)
        sims.append(cosine_similarity(v, quantizer.decompress(quantizer.compress(v, R, n_bits, 32), R)))
    assert np.mean(sims) >= threshold


def test_reference_structure_padding_zero_and_validation():
    R = rotation.generate_rotation_matrix(128, seed=42)
    v = np.random.default_rng(1).standard_normal(128).astype(np.float32)
    c = quantizer.compress(v, R, n_bits=4, group_size=32)
    assert isinstance(c, CompressedKV) and c.quantized_direction.dtype == np.uint8
    assert c.group_mins.shape == (4,) and c.group_scales.shape == (4,) and c.original_dim == 128
    R100 = rotation.generate_rotation_matrix(100, seed=42)
    v100 = np.random.Generator(np.random.PCG64(42)).standard_normal(100).astype(np.float32)
    out = quantizer.decompress(quantizer.compress(v100, R100, 4, 32), R100)
    assert out.shape == (100,) and cosine_similarity(v100, out) >= 0.98
    z = quantizer.compress(np.zeros(128, np.float32), R)
    assert z.radius == 0.0 and np.allclose(quantizer.decompress(z, R), 0.0)
    for bad in (dict(n_bits=1), dict(n_bits=9), dict(group_size=0), dict(group_size=-1), dict(group_size=129)):
        with pytest.raises(ValueError):
            quantizer.compress(v, R, **{"n_bits": 4, "group_size": 32, **bad})


def test_batch_round_trip_and_empty():
    B, H, S, d = 2, 3, 17, 64
    R = rotation.generate_rotation_matrix(d, seed=42)
    kv = np.random.default_rng(3).standard_normal((B, H, S, d)).astype(np.float32)
    comp = quantizer.compress_batch(kv, R, n_bits=4, group_size=32)
    assert len(comp) == B and len(comp[0]) == H and len(comp[0][0]) == S
    one = quantizer.compress(kv[1, 2, 5], R, 4, 32)
    assert comp[1][2][5].radius == one.radius
    assert np.array_equal(comp[1][2][5].quantized_direction, one.quantized_direction)
    out = quantizer.decompress_batch(comp, R)
    assert out.shape == (B, H, S, d) and out.dtype == np.float32
    assert np.array_equal(out[1, 2, 5], quantizer.decompress(one, R))
    empty = quantizer.compress_batch(np.zeros((2, 0, 4, d), np.float32), R)
    assert empty == {"empty": True, "shape": (2, 0, 4, d)}
    assert quantizer.decompress_batch(empty, R).shape == (2, 0, 4, d)
