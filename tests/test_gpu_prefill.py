"""GPU parity of chunked-prefill attention (pqkv_prefill_attn) against the
float64 oracle (oracle.prefill_attention: one decode_attention per query row
with the causal rule), on the same encoded cache bytes.

Tolerance: max |out - oracle| <= 2e-3 and cosine >= 0.9999."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from polarquant_kv import attention, quantizer

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
    return err, cos


def _case(B, Hq, Hkv, Sq, q_start, S, d, seed, kind="normal", S_max=None):
    S_max = S if S_max is None else S_max
    k = O.synth_kv(B, Hkv, S, d, seed + 1, kind)
    v = O.synth_kv(B, Hkv, S, d, seed + 2, kind)
    q = np.random.default_rng(seed).standard_normal((B, Hq, Sq, d)).astype(np.float16)
    R = O.rotation_matrix(d, 42)
    Rt = torch.from_numpy(R.astype(np.float32)).to(DEV)
    kc = quantizer.allocate_cache(B, Hkv, S_max, d, 4, DEV)
    vc = quantizer.allocate_cache(B, Hkv, S_max, d, 4, DEV)
    quantizer.compress_pq(torch.from_numpy(k).to(DEV), Rt, cache=kc)
    quantizer.compress_pq(torch.from_numpy(v).to(DEV), Rt, cache=vc)
    return q, R, Rt, kc, vc


def _oracle(q, R, kc, vc, S, q_start, causal):
    cb = O.lloyd_max_codebook(kc.head_dim, 4)[0]
    kb = kc.blocks.cpu().numpy()[:, :, :S]
    vb = vc.blocks.cpu().numpy()[:, :, :S]
    return O.prefill_attention(q.astype(np.float64), kb, vb, R, cb, cb, q_start=q_start, causal=causal)


CASES = [
    # B, Hq, Hkv, Sq, q_start, S, d, causal, kind
    (1, 8, 2, 16, 48, 64, 128, True, "normal"),          # one q tile, diagonal inside one kv tile
    (1, 16, 2, 100, 156, 256, 128, True, "normal"),      # G=8: 32 tokens per workgroup -> 4 q tiles
    (2, 8, 8, 70, 0, 70, 128, True, "token_ln"),         # G=1, first chunk of the sequence
    (1, 14, 2, 40, 100, 140, 64, True, "normal"),        # G=7: 252 of 256 rows used, d=64
    (1, 12, 4, 33, 0, 300, 64, False, "normal"),         # non-causal, S not a multiple of 64
    (1, 32, 8, 64, 960, 1024, 128, True, "channel"),     # outlier channels: fp32-grade products needed
]


@pytest.mark.parametrize("B,Hq,Hkv,Sq,q0,S,d,causal,kind", CASES,
                         ids=[f"B{c[0]}_Hq{c[1]}_Hkv{c[2]}_Sq{c[3]}_q{c[4]}_S{c[5]}_d{c[6]}_{'c' if c[7] else 'nc'}_{c[8]}"
                              for c in CASES])
def test_prefill_matches_oracle(B, Hq, Hkv, Sq, q0, S, d, causal, kind):
    q, R, Rt, kc, vc = _case(B, Hq, Hkv, Sq, q0, S, d, seed=Sq + S, kind=kind)
    out = attention.prefill_attention(torch.from_numpy(q).to(DEV), kc, vc, Rt, q_start=q0, causal=causal,
                                      out_dtype=torch.float32)
    _check(out.cpu().numpy(), _oracle(q, R, kc, vc, S, q0, causal))


def test_prefill_partial_cache_fp32_query_fp16_out():
    B, Hq, Hkv, Sq, q0, S, d = 1, 8, 2, 24, 76, 100, 128
    q, R, Rt, kc, vc = _case(B, Hq, Hkv, Sq, q0, S, d, seed=3, S_max=160)
    out = attention.prefill_attention(torch.from_numpy(q.astype(np.float32)).to(DEV), kc, vc, Rt, q_start=q0,
                                      causal=True, out_dtype=torch.float16)
    assert out.dtype == torch.float16
    _check(out.float().cpu().numpy(), _oracle(q.astype(np.float32), R, kc, vc, S, q0, True))


def test_prefill_first_row_equals_decode():
    """Causal prefill row i is decode attention over positions <= q_start + i."""
    B, Hq, Hkv, Sq, q0, S, d = 1, 16, 2, 8, 120, 128, 128
    q, R, Rt, kc, vc = _case(B, Hq, Hkv, Sq, q0, S, d, seed=11)
    qt = torch.from_numpy(q).to(DEV)
    pre = attention.prefill_attention(qt, kc, vc, Rt, q_start=q0, causal=True, out_dtype=torch.float32)
    ref = _oracle(q, R, kc, vc, S, q0, True)
    _check(pre.cpu().numpy(), ref)
    # the last row sees the whole cache: the decode kernel on the same cache agrees
    dec = attention.decode_attention(qt[:, :, -1], kc, vc, Rt, out_dtype=torch.float32)
    _check(dec.cpu().numpy(), ref[:, :, -1])


def test_compressed_attention_gpu_multi_token_uses_prefill():
    B, Hq, Hkv, Sq, S, d = 1, 8, 2, 12, 90, 64
    q, R, Rt, kc, vc = _case(B, Hq, Hkv, Sq, S - Sq, S, d, seed=5)
    out = attention.compressed_attention_gpu(torch.from_numpy(q).to(DEV), kc, vc, Rt, causal=True)
    assert out.dtype == torch.float16 and out.shape == (B, Hq, Sq, d)
    _check(out.float().cpu().numpy(), _oracle(q, R, kc, vc, S, S - Sq, True))


def test_prefill_config5_rows_at_full_size():
    """Config 5 shape (64 q / 8 kv heads, d=128, 131072 cached + 2048 new
    tokens, causal): the whole chunk runs on the GPU; rows at the start,
    middle and end of the chunk of one kv-head group are checked against the
    oracle."""
    B, Hq, Hkv, d = 1, 64, 8, 128
    S_cache, Sq = 131072, 2048
    S = S_cache + Sq
    R = O.rotation_matrix(d, 42)
    Rt = torch.from_numpy(R.astype(np.float32)).to(DEV)
    g = torch.Generator(device=DEV)
    g.manual_seed(5)
    kc = quantizer.allocate_cache(B, Hkv, S, d, 4, DEV)
    vc = quantizer.allocate_cache(B, Hkv, S, d, 4, DEV)
    quantizer.compress_pq(torch.randn(B, Hkv, S, d, generator=g, device=DEV).half(), Rt, cache=kc)
    quantizer.compress_pq(torch.randn(B, Hkv, S, d, generator=g, device=DEV).half(), Rt, cache=vc)
    q = torch.randn(B, Hq, Sq, d, generator=g, device=DEV).half()
    out = attention.prefill_attention(q, kc, vc, Rt, q_start=S_cache, causal=True, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    h = 3                                   # kv head; its query heads are 8h .. 8h+7
    cb = O.lloyd_max_codebook(d, 4)[0]
    kb = kc.blocks[:, h:h + 1].cpu().numpy()
    vb = vc.blocks[:, h:h + 1].cpu().numpy()
    qn = q[:, 8 * h:8 * h + 8].cpu().numpy().astype(np.float64)
    for i in (0, 1000, Sq - 1):
        L = S_cache + i + 1
        ref = O.decode_attention(qn[:, :, i], kb[:, :, :L], vb[:, :, :L], R, cb, cb)
        _check(out[:, 8 * h:8 * h + 8, i].cpu().numpy(), ref)
