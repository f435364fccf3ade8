"""Per-token mixed precision on the GPU: pqkv_decode_attn_segments and the
TokenMixedCache built on it, against a float64 softmax over every token of
every segment (the oracle's dequantisation of the same cache bytes)."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from polarquant_kv import attention, policies, quantizer

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _ref_union(q, R, segs, scale=None):
    """q [B, Hq, d] fp16 numpy; segs: list of (k blocks, v blocks, k bits,
    v bits, k codebook, v codebook), blocks [B, Hkv, S_i, bytes]."""
    q = q.astype(np.float64)
    B, Hq, d = q.shape
    ks, vs = [], []
    for kb, vb, kbits, vbits, kcb, vcb in segs:
        if kb.shape[2] == 0:
            continue
        ks.append(O.dequantize_rotated(kb.reshape(-1, kb.shape[-1]), d, kcb, kbits).reshape(*kb.shape[:3], d))
        vs.append(O.dequantize_rotated(vb.reshape(-1, vb.shape[-1]), d, vcb, vbits).reshape(*vb.shape[:3], d))
    k = np.concatenate(ks, axis=2)
    v = np.concatenate(vs, axis=2)
    Hkv = k.shape[1]
    g = Hq // Hkv
    qr = q @ R.T
    scale = 1.0 / np.sqrt(d) if scale is None else scale
    out = np.zeros((B, Hq, d))
    for b in range(B):
        for h in range(Hq):
            s = k[b, h // g] @ qr[b, h] * scale
            p = np.exp(s - s.max())
            out[b, h] = (p / p.sum()) @ v[b, h // g]
    return out @ R


def _check(out, ref):
    err = np.abs(np.asarray(out, np.float64) - ref).max()
    assert err <= 2e-3, err


@pytest.mark.parametrize("case", [(2, 16, 4, 1000, 128), (1, 32, 2, 700, 64), (3, 14, 2, 69, 128)],
                         ids=lambda c: "B{}_Hq{}_Hkv{}_S{}_d{}".format(*c))
def test_token_mixed_cache_attends_on_both_widths(case):
    B, Hq, Hkv, S, d = case
    print(f"token mixed {case}", flush=True)
    rng = np.random.default_rng(S)
    k = O.synth_kv(B, Hkv, S, d, S + 1, "token_ln")
    v = O.synth_kv(B, Hkv, S, d, S + 2, "token_ln")
    q = rng.standard_normal((B, Hq, d)).astype(np.float16)
    R = O.rotation_matrix(d, 42)
    Rt = torch.from_numpy(R.astype(np.float32)).to(DEV)
    tb = policies.compute_token_bitwidths(S)
    cache = policies.TokenMixedCache.from_kv(torch.from_numpy(k).to(DEV), torch.from_numpy(v).to(DEV), Rt, tb)
    assert cache.seq_len == S
    assert abs(cache.avg_bits - tb.double().mean().item()) < 1e-12
    out = cache.attend(torch.from_numpy(q).to(DEV), out_dtype=torch.float32).cpu().numpy()
    segs = []
    for kc, vc, bits in zip(cache.keys, cache.values, cache.bits):
        cb = O.lloyd_max_codebook(d, bits)[0]
        segs.append((kc.blocks.cpu().numpy(), vc.blocks.cpu().numpy(), bits, bits, cb, cb))
    _check(out, _ref_union(q, R, segs))
    # each segment holds its tokens' own encodings: the same bytes as
    # encoding just those positions
    for kc, pos, bits in zip(cache.keys, cache.positions, cache.bits):
        one = quantizer.compress_pq(torch.from_numpy(k[:, :, pos.numpy()]).to(DEV), Rt, bits)
        assert torch.equal(one.blocks, kc.blocks)


def test_decode_segments_widths_capacities_and_an_empty_segment():
    """Three segments of different widths and capacities (S < S_max), one of
    them empty, in one call."""
    B, Hq, Hkv, d = 2, 8, 2, 128
    R = O.rotation_matrix(d, 42)
    Rt = torch.from_numpy(R.astype(np.float32)).to(DEV)
    spec = [(4, 4, 300, 320), (2, 2, 0, 16), (4, 2, 1500, 1600), (2, 4, 77, 77)]
    pairs, segs = [], []
    for i, (kb, vb, S, S_max) in enumerate(spec):
        kc = quantizer.allocate_cache(B, Hkv, S_max, d, kb, DEV)
        vc = quantizer.allocate_cache(B, Hkv, S_max, d, vb, DEV)
        if S:
            quantizer.compress_pq(torch.from_numpy(O.synth_kv(B, Hkv, S, d, 10 + i, "channel")).to(DEV), Rt, cache=kc)
            quantizer.compress_pq(torch.from_numpy(O.synth_kv(B, Hkv, S, d, 20 + i, "channel")).to(DEV), Rt, cache=vc)
        pairs.append((kc, vc))
        segs.append((kc.blocks.cpu().numpy()[:, :, :S], vc.blocks.cpu().numpy()[:, :, :S], kb, vb,
                     O.lloyd_max_codebook(d, kb)[0], O.lloyd_max_codebook(d, vb)[0]))
    q = np.random.default_rng(1).standard_normal((B, Hq, d)).astype(np.float16)
    out = attention.decode_attention_segments(torch.from_numpy(q).to(DEV), pairs, Rt, out_dtype=torch.float32)
    _check(out.cpu().numpy(), _ref_union(q, R, segs))
    # one segment alone is plain decode attention
    one = attention.decode_attention_segments(torch.from_numpy(q).to(DEV), pairs[:1], Rt, out_dtype=torch.float32)
    plain = attention.decode_attention(torch.from_numpy(q).to(DEV), *pairs[0], Rt, out_dtype=torch.float32)
    assert torch.equal(one, plain)


def test_mixed_precision_compress_stats_and_cache():
    B, H, S, d = 1, 2, 200, 128
    kv = torch.from_numpy(O.synth_kv(B, H, S, d, 5, "normal")).to(DEV)
    Rt = torch.from_numpy(O.rotation_matrix(d, 42).astype(np.float32)).to(DEV)
    from polarquant_kv.lloyd_max import get_codebook_torch
    tb = policies.compute_token_bitwidths(S)
    r = policies.mixed_precision_compress(kv, Rt, get_codebook_torch(d, 4, device=DEV),
                                          get_codebook_torch(d, 2, device=DEV), tb)
    assert r["n_high"] == 68 and r["n_low"] == 132
    assert abs(r["avg_bits"] - (68 * 4 + 132 * 2) / 200) < 1e-12
    assert abs(r["compression_ratio"] - 16 / r["avg_bits"]) < 1e-12
    assert torch.equal(r["high_mask"], tb == 4) and torch.equal(r["low_mask"], tb == 2)
    assert r["cache"].seq_len == S and r["cache"].bits == [4, 2]
