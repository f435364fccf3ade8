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


# ---- widths, per-head width maps and the QJL correction ----

def _case_w(B, Hq, Hkv, Sq, q_start, S, d, kbits, vbits, seed, kind="normal", qjl=False):
    k = O.synth_kv(B, Hkv, S, d, seed + 1, kind)
    v = O.synth_kv(B, Hkv, S, d, seed + 2, kind)
    q = np.random.default_rng(seed).standard_normal((B, Hq, Sq, d)).astype(np.float16)
    R = O.rotation_matrix(d, 42)
    Rt = torch.from_numpy(R.astype(np.float32)).to(DEV)
    P = O.jl_matrix(d, d, 43) if qjl else None
    P_rot = torch.from_numpy((P @ R.T).astype(np.float32)).to(DEV) if qjl else None
    kc = quantizer.allocate_cache(B, Hkv, S, d, kbits, DEV, jl_dim=d if qjl else 0)
    vc = quantizer.allocate_cache(B, Hkv, S, d, vbits, DEV)
    quantizer.compress_pq(torch.from_numpy(k).to(DEV), Rt, cache=kc, jl_rot=P_rot)
    quantizer.compress_pq(torch.from_numpy(v).to(DEV), Rt, cache=vc)
    return q, R, Rt, kc, vc, P, P_rot


def _host_blocks(cache, S):
    b = cache.blocks.cpu().numpy()
    if not cache.mixed:
        return b[:, :, :S]
    return [b[:, cache.head_offset(h):cache.head_offset(h) + S * O.vector_bytes(cache.head_dim, bits)]
            .reshape(b.shape[0], S, -1) for h, bits in enumerate(cache.head_bits())]


def _oracle_w(q, R, kc, vc, S, q_start, causal, P=None):
    d = kc.head_dim
    signs = kc.qjl_signs.cpu().numpy()[:, :, :S] if P is not None else None
    kb, vb = _host_blocks(kc, S), _host_blocks(vc, S)
    cbk = [O.lloyd_max_codebook(d, b)[0] for b in kc.head_bits()]
    cbv = [O.lloyd_max_codebook(d, b)[0] for b in vc.head_bits()]
    B, Hq = q.shape[:2]
    Hkv = kc.num_heads
    g = Hq // Hkv
    out = np.zeros(q.shape)
    for h in range(Hkv):
        kh = kb[h] if kc.mixed else kb[:, h]
        vh = vb[h] if vc.mixed else vb[:, h]
        out[:, h * g:(h + 1) * g] = O.prefill_attention(
            q[:, h * g:(h + 1) * g].astype(np.float64), kh[:, None], vh[:, None], R, cbk[h], cbv[h],
            q_start=q_start, causal=causal, k_bits=kc.head_bits()[h], v_bits=vc.head_bits()[h],
            qjl_signs=None if signs is None else signs[:, h:h + 1], P=P)
    return out


WIDTH_CASES = [
    # B, Hq, Hkv, Sq, q_start, S, d, key bits, value bits, causal, qjl
    (1, 8, 2, 40, 100, 140, 128, 2, 2, True, False),
    (1, 16, 2, 70, 0, 200, 128, 4, 2, False, False),
    (2, 6, 3, 33, 67, 100, 64, 2, 4, True, False),
    (1, 8, 2, 48, 80, 128, 128, 4, 4, True, True),       # QJL, 4-bit
    (1, 32, 4, 20, 180, 200, 128, 2, 2, True, True),     # QJL, 2-bit, G = 8 (16 tokens per workgroup)
    (1, 4, 4, 130, 0, 300, 64, 4, 2, False, True),       # QJL, G = 1, d = 64, non-causal
    (1, 8, 2, 16, 48, 64, 128, (4, 2), (2, 4), True, False),               # per-head widths
    (2, 16, 4, 24, 40, 64, 128, (4, 4, 2, 2), (4, 2, 4, 2), True, True),   # four groups, QJL
]


@pytest.mark.parametrize("case", WIDTH_CASES, ids=lambda c: "B{}_Hq{}_Hkv{}_Sq{}_q{}_S{}_d{}_k{}_v{}_{}_{}".format(
    *c[:7], "".join(map(str, np.atleast_1d(c[7]))), "".join(map(str, np.atleast_1d(c[8]))),
    "c" if c[9] else "nc", "qjl" if c[10] else "plain"))
def test_prefill_widths_and_qjl(case):
    B, Hq, Hkv, Sq, q0, S, d, kb, vb, causal, qjl = case
    print(f"prefill widths/qjl case {case}", flush=True)
    q, R, Rt, kc, vc, P, P_rot = _case_w(B, Hq, Hkv, Sq, q0, S, d, kb, vb, seed=Sq + S, kind="channel", qjl=qjl)
    out = attention.prefill_attention(torch.from_numpy(q).to(DEV), kc, vc, Rt, q_start=q0, causal=causal,
                                      out_dtype=torch.float32, jl_rot=P_rot)
    ref = _oracle_w(q, R, kc, vc, S, q0, causal, P=P)
    _check(out.cpu().numpy(), ref)
    if qjl:
        moved = np.abs(_oracle_w(q, R, kc, vc, S, q0, causal) - ref).max()
        print(f"qjl correction moves the output by {moved:.3e}", flush=True)
        assert moved > 2 * MAX_ABS


def test_compressed_attention_gpu_multi_token_with_qjl():
    """The reference applies the QJL term for every query token
    (attention_kernel.py:95-107); compressed_attention_gpu now does too."""
    B, Hq, Hkv, Sq, S, d = 1, 8, 2, 12, 90, 128
    q, R, Rt, kc, vc, P, P_rot = _case_w(B, Hq, Hkv, Sq, S - Sq, S, d, 4, 4, seed=7, qjl=True)
    out = attention.compressed_attention_gpu(torch.from_numpy(q).to(DEV), kc, vc, Rt, jl_matrix=P, causal=True)
    _check(out.float().cpu().numpy(), _oracle_w(q, R, kc, vc, S, S - Sq, True, P=P))


def test_array_api_standard_attention():
    """polarquant_kv.attention.standard_attention on numpy arrays (the
    reference's CPU API name, python/polarquant_kv/attention.py:20-73), 2-D
    and 3-D GQA shapes, against the textbook SDPA; compressed_attention (the
    group format) is checked in test_gpu_group_gpu.py."""
    rng = np.random.default_rng(0)
    d, S = 64, 200
    k2 = rng.standard_normal((S, d)).astype(np.float32)
    v2 = rng.standard_normal((S, d)).astype(np.float32)
    q2 = rng.standard_normal((5, d)).astype(np.float32)
    np.testing.assert_allclose(attention.standard_attention(q2, k2, v2), O.sdpa(q2, k2, v2), atol=1e-5)
    k3 = rng.standard_normal((2, S, d)).astype(np.float32)
    v3 = rng.standard_normal((2, S, d)).astype(np.float32)
    q3 = rng.standard_normal((8, 7, d)).astype(np.float32)
    std3 = attention.standard_attention(q3, k3, v3, num_kv_heads=2)
    want = np.stack([O.sdpa(q3[h], k3[h // 4], v3[h // 4]) for h in range(8)])
    np.testing.assert_allclose(std3, want, atol=1e-5)
    assert not attention.standard_attention(q2, k2[:0], v2[:0]).any()
