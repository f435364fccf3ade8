"""GPU checks on the inputs that pin the oracle's open choices:

- the radius reduction order: the tree probes of test_oracle.py, whose fp32
  radius differs between the reference's 128-slot tree and every other order,
  through the bit-exact quantiser (pqkv_quantize_rotated) and the matrix-core
  encoder (pqkv_encode_mfma, R = I so that the rotated values are the input);
- the QJL rule: a key with a zero residual adds no correction, whether it
  is the zero key or a lossless one; the encoder writes all-ones signs for
  both, and the kernels read an all-ones sketch as a zero residual;
- the saturated fp16 radius: a key whose norm exceeds 65504 is stored as
  65504 and decode stays finite."""

import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from polarquant_kv import _lib, attention, quantizer
from polarquant_kv.lloyd_max import padded_codebook_torch
from polarquant_kv.types import PQCache
from test_oracle import LOSSLESS_IDX, U, lossless_key, qjl_rule_cache, tree_probe

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("d,want_ulps", [(128, 15), (64, 2)])
def test_quantize_rotated_radius_on_tree_probe(d, want_ulps):
    print(f"pins: quantize_rotated tree probe d={d}", flush=True)
    x = np.repeat(tree_probe(d), 3, axis=0)
    x[1] *= np.float32(4.0)                          # scaled by a power of two: same ulps
    c = O.lloyd_max_codebook(d, 4)[0]
    blocks, radius = quantizer.quantize_rotated(torch.from_numpy(x).to(DEV), padded_codebook_torch(d, 4, DEV), 4)
    r = radius.cpu().numpy()
    assert r[0] == np.float32(1.0 + want_ulps * U) and r[2] == r[0]
    assert r[1] == np.float32(4.0 * (1.0 + want_ulps * U))
    want_r, want_idx = O.quantize_rotated(x, c)
    assert np.array_equal(blocks.cpu().numpy(), O.pack_blocks(want_r, want_idx, 4))


@pytest.mark.parametrize("d,want_ulps", [(128, 15), (64, 2)])
@pytest.mark.parametrize("bits", [4, 2])
def test_matrix_core_encoder_radius_on_tree_probe(d, want_ulps, bits):
    """R = I: the matrix-core products with a 0/1 matrix are exact, so the
    rotated values are the fp16 input (1 and 2^-12 are fp16 numbers) and the
    radius is the tree over their squares, computed in the MFMA output
    layout."""
    print(f"pins: encode_mfma tree probe d={d} bits={bits}", flush=True)
    n = 70                                           # more than one 64-vector group
    x = np.repeat(tree_probe(d), n, axis=0).astype(np.float16)
    eye = torch.eye(d, dtype=torch.float32, device=DEV)
    xt = torch.from_numpy(x).to(DEV)
    vb = O.vector_bytes(d, bits)
    blocks = torch.zeros(n, vb, dtype=torch.uint8, device=DEV)
    rot = torch.empty(n, d, dtype=torch.float32, device=DEV)
    rad = torch.empty(n, dtype=torch.float32, device=DEV)
    cb = padded_codebook_torch(d, bits, DEV)
    _lib.check(_lib.lib().pqkv_encode_mfma(xt.data_ptr(), _lib.F16, n * d, eye.data_ptr(), cb.data_ptr(), bits,
                                           blocks.data_ptr(), n * vb, 1, n, d, rot.data_ptr(), rad.data_ptr(),
                                           _lib.stream_of(xt)))
    torch.cuda.synchronize()
    assert np.array_equal(rot.cpu().numpy(), x.astype(np.float32))
    assert (rad.cpu().numpy() == np.float32(1.0 + want_ulps * U)).all()
    r, idx = O.quantize_rotated(x.astype(np.float32), O.lloyd_max_codebook(d, bits)[0])
    assert np.array_equal(blocks.cpu().numpy(), O.pack_blocks(r, idx, bits))


@pytest.mark.parametrize("d", [64, 128])
def test_exact_encoder_signs_of_zero_and_lossless_keys(d):
    """fp32 input through pqkv_encode with R = I (the FMA chain against a 0/1
    matrix is exact) and QJL: the zero key and the lossless key have residual
    0, so all their signs are 1 (P 0 = 0 >= 0); their blocks are the
    oracle's."""
    print(f"pins: exact encoder QJL zero/lossless keys d={d}", flush=True)
    rng = np.random.default_rng(d)
    x = rng.standard_normal((5, d)).astype(np.float32)
    x[0] = 0.0
    x[1] = lossless_key(d)
    x[3] = lossless_key(d, scale=0.5)
    eye = torch.eye(d, dtype=torch.float32, device=DEV)
    P = torch.from_numpy(O.jl_matrix(d, d, 43).astype(np.float32)).to(DEV)    # P R^T with R = I
    kc = quantizer.compress_pq(torch.from_numpy(x[None, None]).to(DEV), eye, 4, jl_rot=P)
    torch.cuda.synchronize()
    signs = kc.qjl_signs.cpu().numpy()[0, 0]
    assert (signs[[0, 1, 3]] == 0xFF).all()
    c = O.lloyd_max_codebook(d, 4)[0]
    r, idx = O.quantize_rotated(x, c)
    assert r[1] == np.float32(2.0) and np.array_equal(idx[1], LOSSLESS_IDX[d])
    assert np.array_equal(kc.blocks.cpu().numpy()[0, 0], O.pack_blocks(r, idx, 4))


def _cache_from_host(blocks, d, bits, signs=None):
    B, H, S, _ = blocks.shape
    return PQCache(blocks=torch.from_numpy(np.ascontiguousarray(blocks)).to(DEV), head_dim=d, n_bits=bits,
                   seq_len=S, max_seq_len=S, codebooks=padded_codebook_torch(d, bits, DEV),
                   qjl_signs=None if signs is None else torch.from_numpy(np.ascontiguousarray(signs)).to(DEV),
                   jl_dim=0 if signs is None else d)


@pytest.mark.parametrize("d", [64, 128])
def test_decode_qjl_rule_zero_and_lossless_keys(d):
    """Decode on the rule cache: within 2e-3 of the oracle (pinned by hand in
    test_oracle.py: zero-residual keys, i.e. all-ones sketches, get no
    correction), and the two other rules (no guard at all; a guard on the
    radius only) land far outside that tolerance on this input."""
    print(f"pins: decode QJL rule d={d}", flush=True)
    S, G = 6, 4
    kb, vb, signs, P, R, c, _ = qjl_rule_cache(d, S, key_scale=0.1)
    # queries along P^T 1, where the all-ones correction (1/m) sum_i (P q)_i
    # is largest, so each rule moves the scores by O(1)
    a = P.T @ np.ones(d)
    rng = np.random.default_rng(5)
    q = np.stack([80.0 * (a / np.linalg.norm(a) + 0.1 * rng.standard_normal(d)) for _ in range(G)])
    q = q[None].astype(np.float32)
    Rt = torch.from_numpy(R.astype(np.float32)).to(DEV)
    P_rot = torch.from_numpy((P @ R.T).astype(np.float32)).to(DEV)
    kc = _cache_from_host(kb, d, 4, signs)
    vc = _cache_from_host(vb, d, 4)
    out = attention.decode_attention(torch.from_numpy(q).to(DEV), kc, vc, Rt, jl_rot=P_rot,
                                     out_dtype=torch.float32).cpu().numpy().astype(np.float64)
    ref = O.decode_attention(q.astype(np.float64), kb, vb, R, c, c, qjl_signs=signs, P=P)
    assert np.abs(out - ref).max() <= 2e-3

    # the other rules, by the same hand formula as the oracle test
    r16, idx = O.unpack_blocks(kb[0, 0], d, 4)
    K = r16.astype(np.float64)[:, None] * c[idx].astype(np.float64)
    Vr = O.dequantize_rotated(vb[0, 0], d, c)
    bits = O.bit_unpack_lsb(signs[0, 0], d).astype(np.float64) * 2 - 1
    scale = 1 / math.sqrt(d)

    def rule_out(corrected):
        o = np.zeros((1, G, d))
        for g in range(G):
            qr, pq = R @ q[0, g], P @ q[0, g]
            s = np.array([qr @ K[t] + (bits[t] @ pq / d if corrected(t) else 0.0) for t in range(S)]) * scale
            w = np.exp(s - s.max())
            o[0, g] = ((w / w.sum()) @ Vr) @ R
        return o

    np.testing.assert_allclose(rule_out(lambda t: t > 1), ref, atol=1e-9)
    for other in (lambda t: True, lambda t: t != 0):
        assert np.abs(rule_out(other) - out).max() > 25 * 2e-3


def test_decode_with_radius_past_fp16_range_is_finite():
    """A key and a value of norm ~1.2e5: stored radius 65504 (0x7BFF), output
    finite and within tolerance of the oracle on the same bytes."""
    print("pins: saturated radius decode", flush=True)
    B, Hq, Hkv, S, d = 1, 4, 1, 40, 128
    rng = np.random.default_rng(9)
    k = rng.standard_normal((B, Hkv, S, d)).astype(np.float16)
    v = rng.standard_normal((B, Hkv, S, d)).astype(np.float16)
    k[0, 0, 7, :4] = 60000.0
    v[0, 0, 11, :4] = -60000.0
    R = O.rotation_matrix(d, 42)
    Rt = torch.from_numpy(R.astype(np.float32)).to(DEV)
    kc = quantizer.compress_pq(torch.from_numpy(k).to(DEV), Rt)
    vc = quantizer.compress_pq(torch.from_numpy(v).to(DEV), Rt)
    kb, vb = kc.blocks.cpu().numpy(), vc.blocks.cpu().numpy()
    for blk, t in ((kb, 7), (vb, 11)):
        assert blk[0, 0, t, 0] == 0xFF and blk[0, 0, t, 1] == 0x7B
    q = (0.01 * rng.standard_normal((B, Hq, d))).astype(np.float16)
    out = attention.decode_attention(torch.from_numpy(q).to(DEV), kc, vc, Rt, out_dtype=torch.float32)
    got = out.cpu().numpy().astype(np.float64)
    assert np.isfinite(got).all()
    c = O.lloyd_max_codebook(d, 4)[0]
    ref = O.decode_attention(q.astype(np.float64), kb, vb, R, c, c)
    assert np.abs(got - ref).max() <= 2e-3 * max(1.0, np.abs(ref).max() / 100)
