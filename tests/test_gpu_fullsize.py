"""Parity at each BASELINE configuration's real size (configs 2, 3 and 4).

The whole batch runs on the GPU at the configuration's shape and data law;
the oracle (float64) checks a few (batch, kv-head) streams of the same
cache bytes, and every output row must be finite. The exact encoder is
bit-checked on a sample of a full-size tensor, and the matrix-core encoder's
quantiser on a sample of its own full-size rotation."""

import numpy as np
import pytest
import torch

import oracle as OC
from oracle import oracle as O
from polarquant_kv import _lib, attention, quantizer
from polarquant_kv.lloyd_max import padded_codebook_torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
MAX_ABS = 2e-3
MIN_COS = 0.9999


def _check(out, ref):
    out = np.asarray(out, np.float64)
    err = np.abs(out - ref).max()
    cos = (out * ref).sum() / (np.linalg.norm(out) * np.linalg.norm(ref) + 1e-300)
    assert err <= MAX_ABS, f"max abs err {err}"
    assert cos >= MIN_COS, f"cosine {cos}"


def _token_lognormal(B, H, S, d, seed):
    """N(0,1) with each token's vector scaled by LogNormal(0, 0.5) (config 2)."""
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    x = torch.randn(B, H, S, d, generator=g, device=DEV)
    return (x * torch.exp(0.5 * torch.randn(B, H, S, 1, generator=g, device=DEV))).half()


def _channel_law(B, H, S, d, seed):
    """Per-(head, channel) std LogNormal(0, 1), 1 % of the channels x20
    (configs 3 and 4)."""
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    std = torch.exp(torch.randn(1, H, 1, d, generator=g, device=DEV))
    n_out = max(1, round(0.01 * d))
    for h in range(H):
        std[0, h, 0, torch.randperm(d, generator=g, device=DEV)[:n_out]] *= 20.0
    x = torch.randn(B, H, S, d, generator=g, device=DEV)
    return (x * std).clamp_(-65504, 65504).half()


def _encode_rows(make, B, H, S, d, bits, seed, jl_rot=None):
    """A [B, H, S] cache filled one batch row at a time (bounded staging)."""
    R = torch.from_numpy(O.rotation_matrix(d, 42).astype(np.float32)).to(DEV)
    c = quantizer.allocate_cache(B, H, S, d, bits, DEV, jl_dim=d if jl_rot is not None else 0)
    for b in range(B):
        sub = quantizer.allocate_cache(1, H, S, d, bits, DEV, jl_dim=d if jl_rot is not None else 0)
        quantizer.compress_pq(make(1, H, S, d, seed + 1000 * b), R, cache=sub, jl_rot=jl_rot)
        c.blocks[b] = sub.blocks[0]
        if jl_rot is not None:
            c.qjl_signs[b] = sub.qjl_signs[0]
    c.seq_len = S
    return c, R


def _stream(cache, b, h, S):
    """Host bytes of stream (b, h): [1, 1, S, vector bytes]."""
    blk = cache.blocks[b].cpu().numpy()
    if cache.mixed:
        vb = O.vector_bytes(cache.head_dim, cache.head_bits()[h])
        off = cache.head_offset(h)
        return blk[off:off + S * vb].reshape(1, 1, S, vb)
    return blk[h:h + 1, :S][None]


def _oracle_stream(q, R, kc, vc, b, h, g, S, P=None):
    d = kc.head_dim
    kb, vb = kc.head_bits()[h], vc.head_bits()[h]
    signs = None
    if P is not None:
        signs = kc.qjl_signs[b:b + 1, h:h + 1, :S].cpu().numpy()
    return O.decode_attention(q[b:b + 1, g * h:g * h + g].astype(np.float64), _stream(kc, b, h, S),
                              _stream(vc, b, h, S), R, O.lloyd_max_codebook(d, kb)[0],
                              O.lloyd_max_codebook(d, vb)[0], k_bits=kb, v_bits=vb, qjl_signs=signs, P=P)


def test_config2_full_size():
    """B=16, 14 q / 2 kv heads, d=64, S=4096, 4-bit K and V, per-token
    LogNormal(0, 0.5) norms."""
    B, Hq, Hkv, S, d = 16, 14, 2, 4096, 64
    print("config 2 full size", flush=True)
    kc, Rt = _encode_rows(_token_lognormal, B, Hkv, S, d, 4, 21)
    vc, _ = _encode_rows(_token_lognormal, B, Hkv, S, d, 4, 22)
    q = np.random.default_rng(2).standard_normal((B, Hq, d)).astype(np.float16)
    out = attention.decode_attention(torch.from_numpy(q).to(DEV), kc, vc, Rt, out_dtype=torch.float32)
    out = out.cpu().numpy()
    assert np.isfinite(out).all()
    R, g = O.rotation_matrix(d, 42), Hq // Hkv
    for b, h in ((0, 0), (7, 1), (15, 0), (11, 1)):
        _check(out[b:b + 1, g * h:g * h + g], _oracle_stream(q, R, kc, vc, b, h, g, S))


def test_config3_full_size_channel_law():
    """B=8, 32 q / 8 kv heads, d=128, S=32768, 4-bit, the configuration's
    per-channel LogNormal(0, 1) stds with 1 % outlier channels x20."""
    B, Hq, Hkv, S, d = 8, 32, 8, 32768, 128
    print("config 3 full size, channel law", flush=True)
    kc, Rt = _encode_rows(_channel_law, B, Hkv, S, d, 4, 31)
    vc, _ = _encode_rows(_channel_law, B, Hkv, S, d, 4, 32)
    q = np.random.default_rng(3).standard_normal((B, Hq, d)).astype(np.float16)
    out = attention.decode_attention(torch.from_numpy(q).to(DEV), kc, vc, Rt, out_dtype=torch.float32)
    out = out.cpu().numpy()
    assert np.isfinite(out).all()
    R, g = O.rotation_matrix(d, 42), Hq // Hkv
    for b, h in ((0, 0), (3, 5), (7, 7), (5, 2)):
        _check(out[b:b + 1, g * h:g * h + g], _oracle_stream(q, R, kc, vc, b, h, g, S))


@pytest.mark.parametrize("widths", ["all2", "mixed"])
def test_config4_full_size_qjl(widths):
    """B=4, 32 q / 8 kv heads, d=128, S=16384, QJL on the keys: all heads
    2-bit, or per-head 4/2-bit codebooks (4, 2, 2, 4, 2, 4, 4, 2)."""
    B, Hq, Hkv, S, d = 4, 32, 8, 16384, 128
    print(f"config 4 full size {widths}", flush=True)
    bits = 2 if widths == "all2" else (4, 2, 2, 4, 2, 4, 4, 2)
    R = O.rotation_matrix(d, 42)
    P = O.jl_matrix(d, d, 43)
    P_rot = torch.from_numpy((P @ R.T).astype(np.float32)).to(DEV)
    kc, Rt = _encode_rows(_channel_law, B, Hkv, S, d, bits, 41, jl_rot=P_rot)
    vc, _ = _encode_rows(_channel_law, B, Hkv, S, d, bits, 42)
    q = np.random.default_rng(4).standard_normal((B, Hq, d)).astype(np.float16)
    out = attention.decode_attention(torch.from_numpy(q).to(DEV), kc, vc, Rt, jl_rot=P_rot, out_dtype=torch.float32)
    out = out.cpu().numpy()
    assert np.isfinite(out).all()
    g = Hq // Hkv
    for b, h in ((0, 0), (1, 3), (3, 6), (2, 7)):
        _check(out[b:b + 1, g * h:g * h + g], _oracle_stream(q, R, kc, vc, b, h, g, S, P=P))


def test_config3_exact_encode_sample_bit_exact(monkeypatch):
    """The exact encoder on a whole config-3 K tensor (2 097 152 vectors):
    a sample of 4096 vectors spread over it equals the oracle's FMA-chain
    rotation -> quantiser -> packing, bit for bit."""
    monkeypatch.setenv("PQKV_ENCODE_KERNEL", "exact")
    B, Hkv, S, d = 8, 8, 32768, 128
    print("config 3 exact encode sample", flush=True)
    kc, _ = _encode_rows(_channel_law, B, Hkv, S, d, 4, 31)
    R32 = O.rotation_matrix(d, 42).astype(np.float32)
    idx = np.random.default_rng(5).choice(B * Hkv * S, 4096, replace=False)
    x = torch.cat([_channel_law(1, Hkv, S, d, 31 + 1000 * b) for b in range(B)]).reshape(-1, d)
    xs = x[torch.from_numpy(idx).to(DEV)].float().cpu().numpy()
    got = kc.blocks.reshape(-1, 72)[torch.from_numpy(idx).to(DEV)].cpu().numpy()
    rot = OC.c_rotate_fma(xs, R32)
    r, codes = OC.c_quantize_rotated(rot, O.lloyd_max_codebook(d, 4)[0])
    assert np.array_equal(got, OC.c_pack_blocks(r, codes, 4))


def test_config3_mfma_encode_sample_on_its_rotation():
    """The matrix-core encoder on a whole config-3 K tensor: a sample of
    4096 vectors' blocks equal the oracle quantiser on the rotation the
    encoder returns for them."""
    B, Hkv, S, d = 8, 8, 32768, 128
    print("config 3 mfma encode sample", flush=True)
    x = torch.cat([_channel_law(1, Hkv, S, d, 31 + 1000 * b) for b in range(B)]).reshape(-1, d)
    n = x.shape[0]
    R32 = O.rotation_matrix(d, 42).astype(np.float32)
    Rt = torch.from_numpy(R32).to(DEV)
    blocks = torch.zeros(n, 72, dtype=torch.uint8, device=DEV)
    rot = torch.empty(n, d, dtype=torch.float32, device=DEV)
    _lib.check(_lib.lib().pqkv_encode_mfma(x.data_ptr(), _lib.F16, n * d, Rt.data_ptr(),
                                           padded_codebook_torch(d, 4, DEV).data_ptr(), 4, blocks.data_ptr(),
                                           n * 72, 1, n, d, rot.data_ptr(), None, _lib.stream_of(x)))
    torch.cuda.synchronize()
    idx = torch.from_numpy(np.random.default_rng(6).choice(n, 4096, replace=False)).to(DEV)
    r, codes = OC.c_quantize_rotated(rot[idx].cpu().numpy(), O.lloyd_max_codebook(d, 4)[0])
    assert np.array_equal(blocks[idx].cpu().numpy(), OC.c_pack_blocks(r, codes, 4))
