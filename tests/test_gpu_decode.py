"""GPU parity of decode attention against the float64 oracle.

Tolerance: max |out - oracle| <= 2e-3 and
cosine(out, oracle) >= 0.9999, on the same encoded cache (the cache is
encoded on the GPU, copied back and handed to the oracle byte for byte)."""

import math

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


def _setup(B, Hq, Hkv, S, d, kbits, vbits, seed, S_max=None, kind="token_ln", qjl=False):
    S_max = S if S_max is None else S_max
    rng = np.random.default_rng(seed)
    k = O.synth_kv(B, Hkv, S, d, seed + 1, kind)
    v = O.synth_kv(B, Hkv, S, d, seed + 2, kind)
    q = rng.standard_normal((B, Hq, d)).astype(np.float16)
    R = O.rotation_matrix(d, 42)
    Rt = torch.from_numpy(R.astype(np.float32)).to(DEV)
    P_rot = None
    if qjl:
        P = O.jl_matrix(d, d, 43)
        P_rot = torch.from_numpy((P @ R.T).astype(np.float32)).to(DEV)
    kc = quantizer.allocate_cache(B, Hkv, S_max, d, kbits, DEV, jl_dim=d if qjl else 0)
    vc = quantizer.allocate_cache(B, Hkv, S_max, d, vbits, DEV)
    if S:
        quantizer.compress_pq(torch.from_numpy(k).to(DEV), Rt, cache=kc, jl_rot=P_rot)
        quantizer.compress_pq(torch.from_numpy(v).to(DEV), Rt, cache=vc)
    return q, R, Rt, kc, vc, P_rot


def _host_blocks(cache, S):
    """[B, H, S, bytes] per head (mixed widths: list of per-head arrays)."""
    b = cache.blocks.cpu().numpy()
    if not cache.mixed:
        return b[:, :, :S]
    out = []
    for h, bits in enumerate(cache.head_bits()):
        vb = O.vector_bytes(cache.head_dim, bits)
        off = cache.head_offset(h)
        out.append(b[:, off:off + S * vb].reshape(b.shape[0], S, vb))
    return out


def _oracle(q, R, kc, vc, S, P=None, signs=None):
    d = kc.head_dim
    cbk = [O.lloyd_max_codebook(d, bb)[0] for bb in kc.head_bits()]
    cbv = [O.lloyd_max_codebook(d, bb)[0] for bb in vc.head_bits()]
    kb, vb = _host_blocks(kc, S), _host_blocks(vc, S)
    if kc.mixed or vc.mixed:
        B, Hq = q.shape[:2]
        Hkv = kc.num_heads
        g = Hq // Hkv
        out = np.zeros(q.shape)
        for h in range(Hkv):
            kh = kb[h] if kc.mixed else kb[:, h]
            vh = vb[h] if vc.mixed else vb[:, h]
            out[:, h * g:(h + 1) * g] = O.decode_attention(
                q[:, h * g:(h + 1) * g].astype(np.float64), kh[:, None], vh[:, None], R, cbk[h], cbv[h],
                k_bits=kc.head_bits()[h], v_bits=vc.head_bits()[h],
                qjl_signs=None if signs is None else signs[:, h:h + 1], P=P)
        return out
    return O.decode_attention(q.astype(np.float64), kb, vb, R, cbk[0], cbv[0], k_bits=kc.head_bits()[0],
                              v_bits=vc.head_bits()[0], qjl_signs=signs, P=P)


CASES = [
    # B, Hq, Hkv, S, d, kbits, vbits
    (1, 14, 2, 512, 64, 4, 4),      # config 1 shape (Qwen2.5-0.5B layer)
    (2, 32, 8, 300, 128, 4, 4),     # 8B shape, short
    (1, 8, 8, 100, 128, 4, 4),      # G = 1 (MHA, the reference benchmark's heads)
    (1, 16, 2, 129, 128, 4, 4),     # G = 8
    (2, 12, 4, 65, 64, 4, 4),       # G = 3, tile + 1
    (1, 4, 2, 1, 128, 4, 4),        # one token
    (1, 4, 1, 64, 128, 2, 2),       # 2-bit
    (2, 8, 2, 200, 128, 4, 2),      # 4-bit K, 2-bit V
    (1, 6, 2, 77, 64, 2, 4),        # 2-bit K, 4-bit V
    (1, 8, 1, 1500, 64, 2, 2),      # several splits
    (1, 32, 2, 300, 128, 4, 4),     # G = 16: two launches of 8 query heads per kv head
    (2, 12, 1, 200, 64, 4, 2),      # G = 12: two launches of 6
    (1, 9, 1, 130, 128, 2, 2),      # G = 9: launches of 5 and 4
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}_Hq{}_Hkv{}_S{}_d{}_k{}v{}".format(*c))
def test_decode_matches_oracle(case):
    B, Hq, Hkv, S, d, kb, vb = case
    print(f"decode case {case}", flush=True)
    q, R, Rt, kc, vc, _ = _setup(B, Hq, Hkv, S, d, kb, vb, seed=sum(case))
    out = attention.decode_attention(torch.from_numpy(q).to(DEV), kc, vc, Rt, out_dtype=torch.float32)
    ref = _oracle(q, R, kc, vc, S)
    _check(out.cpu().numpy(), ref)


VALU_CASES = [c for c in CASES if c[5] == 4 and c[6] == 4][:4]


@pytest.mark.parametrize("case", VALU_CASES, ids=lambda c: "B{}_Hq{}_Hkv{}_S{}_d{}_k{}v{}".format(*c))
def test_decode_valu_kernel_matches_oracle(case, monkeypatch):
    """The fp32 VALU kernel on 4-bit caches (the matrix-core kernel serves
    them by default)."""
    monkeypatch.setenv("PQKV_DECODE_KERNEL", "valu")
    B, Hq, Hkv, S, d, kb, vb = case
    q, R, Rt, kc, vc, _ = _setup(B, Hq, Hkv, S, d, kb, vb, seed=sum(case) + 1)
    out = attention.decode_attention(torch.from_numpy(q).to(DEV), kc, vc, Rt, out_dtype=torch.float32)
    _check(out.cpu().numpy(), _oracle(q, R, kc, vc, S))


@pytest.mark.parametrize("same_content", [True, False], ids=["copy", "scaled"])
def test_decode_value_codebook_of_its_own(same_content):
    """4-bit keys and values whose codebooks sit at different addresses: the
    values read their own table (keys and values share one table only when
    they pass the same codebook pointer). A scaled value codebook shows that
    the values really use theirs."""
    from polarquant_kv.lloyd_max import padded_codebook_torch
    B, Hq, Hkv, S, d = 2, 16, 4, 600, 128
    cbk = padded_codebook_torch(d, 4, DEV)
    cbv = cbk.clone() if same_content else cbk * 0.9
    rng = np.random.default_rng(5)
    k = O.synth_kv(B, Hkv, S, d, 6, "token_ln")
    v = O.synth_kv(B, Hkv, S, d, 7, "token_ln")
    q = rng.standard_normal((B, Hq, d)).astype(np.float16)
    R = O.rotation_matrix(d, 42)
    Rt = torch.from_numpy(R.astype(np.float32)).to(DEV)
    kc = quantizer.allocate_cache(B, Hkv, S, d, 4, DEV)
    vc = quantizer.allocate_cache(B, Hkv, S, d, 4, DEV, codebooks=cbv)
    assert kc.codebooks.data_ptr() != vc.codebooks.data_ptr()
    quantizer.compress_pq(torch.from_numpy(k).to(DEV), Rt, cache=kc)
    quantizer.compress_pq(torch.from_numpy(v).to(DEV), Rt, cache=vc)
    out = attention.decode_attention(torch.from_numpy(q).to(DEV), kc, vc, Rt, out_dtype=torch.float32)
    ref = O.decode_attention(q.astype(np.float64), kc.blocks.cpu().numpy()[:, :, :S], vc.blocks.cpu().numpy()[:, :, :S],
                             R, cbk.cpu().numpy()[:16].astype(np.float64), cbv.cpu().numpy()[:16].astype(np.float64),
                             k_bits=4, v_bits=4)
    _check(out.cpu().numpy(), ref)


def test_decode_outlier_channels_both_kernels(monkeypatch):
    """The metric config's data law (per-channel LogNormal std, 1 % of the
    channels x20): outputs reach ~1e2, so this is the case that needs
    fp32-grade arithmetic in both kernels."""
    B, Hq, Hkv, S, d = 2, 32, 8, 700, 128
    q, R, Rt, kc, vc, _ = _setup(B, Hq, Hkv, S, d, 4, 4, seed=77, kind="channel")
    ref = _oracle(q, R, kc, vc, S)
    assert np.abs(ref).max() > 10.0
    for kernel in ("mfma", "valu"):
        monkeypatch.setenv("PQKV_DECODE_KERNEL", kernel)
        out = attention.decode_attention(torch.from_numpy(q).to(DEV), kc, vc, Rt, out_dtype=torch.float32)
        _check(out.cpu().numpy(), ref)


def test_decode_partial_cache_and_dtypes():
    # S < S_max, fp32 query, fp16 output
    q, R, Rt, kc, vc, _ = _setup(2, 8, 2, 700, 128, 4, 4, seed=5, S_max=1000)
    qf = torch.from_numpy(q.astype(np.float32)).to(DEV)
    out = attention.decode_attention(qf, kc, vc, Rt, out_dtype=torch.float16)
    assert out.dtype == torch.float16
    _check(out.float().cpu().numpy(), _oracle(q.astype(np.float32), R, kc, vc, 700))


def test_decode_empty_cache_gives_zeros():
    q, R, Rt, kc, vc, _ = _setup(1, 4, 2, 0, 128, 4, 4, seed=1, S_max=8)
    out = attention.decode_attention(torch.from_numpy(q).to(DEV), kc, vc, Rt)
    assert torch.count_nonzero(out).item() == 0


MIXED_CASES = [
    # key widths, value widths, QJL
    ((4, 4, 4, 4, 2, 2, 2, 2), (4, 4, 4, 4, 2, 2, 2, 2), False),   # 4/4 + 2/2: one launch
    ((2, 4, 2, 4, 4, 2, 2, 4), (2, 4, 2, 4, 4, 2, 2, 4), True),    # the same, interleaved, QJL
    ((4, 4, 2, 2, 4, 2, 4, 2), (2, 4, 2, 4, 4, 4, 2, 2), False),   # four groups: a launch each
]


@pytest.mark.parametrize("case", MIXED_CASES, ids=["pair", "pair_interleaved_qjl", "four_groups"])
def test_decode_mixed_widths(case):
    kw_, vw_, qjl = case
    B, Hq, Hkv, S, d = 2, 32, 8, 1400, 128
    print(f"mixed case {case}", flush=True)
    rng = np.random.default_rng(12)
    k = O.synth_kv(B, Hkv, S, d, 31, "channel")
    v = O.synth_kv(B, Hkv, S, d, 32, "channel")
    q = rng.standard_normal((B, Hq, d)).astype(np.float16)
    R = O.rotation_matrix(d, 42)
    Rt = torch.from_numpy(R.astype(np.float32)).to(DEV)
    P = O.jl_matrix(d, d, 43) if qjl else None
    P_rot = torch.from_numpy((P @ R.T).astype(np.float32)).to(DEV) if qjl else None
    kc = quantizer.allocate_cache(B, Hkv, S, d, kw_, DEV, jl_dim=d if qjl else 0)
    vc = quantizer.allocate_cache(B, Hkv, S, d, vw_, DEV)
    quantizer.compress_pq(torch.from_numpy(k).to(DEV), Rt, cache=kc, jl_rot=P_rot)
    quantizer.compress_pq(torch.from_numpy(v).to(DEV), Rt, cache=vc)
    kw = dict(jl_rot=P_rot) if qjl else {}
    out = attention.decode_attention(torch.from_numpy(q).to(DEV), kc, vc, Rt, out_dtype=torch.float32, **kw)
    signs = kc.qjl_signs.cpu().numpy()[:, :, :S] if qjl else None
    _check(out.cpu().numpy(), _oracle(q, R, kc, vc, S, P=P, signs=signs))


QJL_CASES = [
    # B, Hq, Hkv, S, d, kbits, vbits
    (1, 8, 2, 300, 128, 2, 2),      # config 4 shape family (G = 4)
    (1, 16, 2, 333, 128, 4, 4),     # G = 8: whole-chunk reloads, one shared 4-bit table
    (2, 14, 2, 257, 64, 4, 2),      # G = 7, d = 64, 4-bit K / 2-bit V
    (1, 4, 4, 100, 128, 4, 4),      # G = 1
    (1, 40, 2, 150, 128, 2, 2),     # G = 20: launches of 7, 7 and 6
]


@pytest.mark.parametrize("case", QJL_CASES, ids=lambda c: "B{}_Hq{}_Hkv{}_S{}_d{}_k{}v{}".format(*c))
def test_decode_qjl_correction(case):
    B, Hq, Hkv, S, d, kb, vb = case
    print(f"qjl case {case}", flush=True)
    q, R, Rt, kc, vc, P_rot = _setup(B, Hq, Hkv, S, d, kb, vb, seed=21 + sum(case), qjl=True)
    out = attention.decode_attention(torch.from_numpy(q).to(DEV), kc, vc, Rt, jl_rot=P_rot,
                                     out_dtype=torch.float32)
    P = O.jl_matrix(d, d, 43)
    signs = kc.qjl_signs.cpu().numpy()[:, :, :S]
    ref = _oracle(q, R, kc, vc, S, P=P, signs=signs)
    _check(out.cpu().numpy(), ref)
    # the correction must matter: without it the result moves (1.2e-2 to
    # 2.7e-2 on these cases)
    plain = _oracle(q, R, kc, vc, S)
    moved = np.abs(plain - ref).max()
    print(f"qjl correction moves the output by {moved:.3e}", flush=True)
    assert moved > 2 * MAX_ABS


def test_compressed_attention_gpu_api():
    q, R, Rt, kc, vc, _ = _setup(1, 14, 2, 256, 64, 4, 4, seed=2)
    q4 = torch.from_numpy(q).to(DEV).unsqueeze(2)        # [B, Hq, 1, d]
    out = attention.compressed_attention_gpu(q4, kc, vc, Rt, num_kv_heads=2)
    assert out.shape == q4.shape and out.dtype == torch.float16
    _check(out[:, :, 0].float().cpu().numpy(), _oracle(q, R, kc, vc, 256))


def test_decode_full_size_config3_slices():
    """Config 3 at its real shape (B=8, Hq=32, Hkv=8, d=128, S=32768): the
    whole batch runs on the GPU; four (batch, kv-head) streams are checked
    against the oracle and the output rows are all finite with unit-scale
    norms."""
    B, Hq, Hkv, S, d = 8, 32, 8, 32768, 128
    torch.manual_seed(0)
    R = O.rotation_matrix(d, 42)
    Rt = torch.from_numpy(R.astype(np.float32)).to(DEV)
    kc = quantizer.allocate_cache(B, Hkv, S, d, 4, DEV)
    vc = quantizer.allocate_cache(B, Hkv, S, d, 4, DEV)
    for b in range(B):   # encode one batch row at a time to bound the fp16 staging
        k = torch.randn(1, Hkv, S, d, device=DEV, dtype=torch.float16)
        v = torch.randn(1, Hkv, S, d, device=DEV, dtype=torch.float16)
        sub_k = quantizer.allocate_cache(1, Hkv, S, d, 4, DEV)
        sub_v = quantizer.allocate_cache(1, Hkv, S, d, 4, DEV)
        quantizer.compress_pq(k, Rt, cache=sub_k)
        quantizer.compress_pq(v, Rt, cache=sub_v)
        kc.blocks[b] = sub_k.blocks[0]
        vc.blocks[b] = sub_v.blocks[0]
    kc.seq_len = vc.seq_len = S
    q = torch.randn(B, Hq, d, device=DEV, dtype=torch.float16)
    out = attention.decode_attention(q, kc, vc, Rt, out_dtype=torch.float32).cpu().numpy()
    assert np.isfinite(out).all()
    qn = q.cpu().numpy()
    kb = kc.blocks.cpu().numpy()
    vb = vc.blocks.cpu().numpy()
    cb = O.lloyd_max_codebook(d, 4)[0]
    for b, h in ((0, 0), (3, 5), (7, 7), (5, 2)):
        ref = O.decode_attention(qn[b:b + 1, 4 * h:4 * h + 4].astype(np.float64), kb[b:b + 1, h:h + 1],
                                 vb[b:b + 1, h:h + 1], R, cb, cb)
        _check(out[b:b + 1, 4 * h:4 * h + 4], ref)


def test_decode_workspace_any_contents_and_reuse():
    """A workspace full of random bytes, reused across calls and across
    shapes (different split plans), gives the same bits every time and
    matches the oracle: nothing is read from it before being written."""
    cases = [((2, 16, 4, 3000, 128, 4, 4), False), ((1, 8, 2, 1777, 128, 2, 2), True),
             ((2, 16, 4, 900, 128, 4, 4), False)]
    need = max(_lib_decode_bytes(c[0]) for c in cases)
    ws = torch.randint(0, 256, (need,), dtype=torch.uint8, device=DEV)
    for case, qjl in cases:
        B, Hq, Hkv, S, d, kb, vb = case
        print(f"workspace reuse case {case} qjl={qjl}", flush=True)
        q, R, Rt, kc, vc, P_rot = _setup(B, Hq, Hkv, S, d, kb, vb, seed=S, qjl=qjl)
        qt = torch.from_numpy(q).to(DEV)
        kw = dict(jl_rot=P_rot) if qjl else {}
        outs = [attention.decode_attention(qt, kc, vc, Rt, out_dtype=torch.float32, workspace=ws, **kw)
                for _ in range(3)]
        for o in outs[1:]:
            assert torch.equal(o, outs[0])
        if qjl:
            ref = _oracle(q, R, kc, vc, S, P=O.jl_matrix(d, d, 43), signs=kc.qjl_signs.cpu().numpy()[:, :, :S])
        else:
            ref = _oracle(q, R, kc, vc, S)
        _check(outs[0].cpu().numpy(), ref)


def _lib_decode_bytes(case):
    from polarquant_kv import _lib
    B, Hq, Hkv, S, d = case[:5]
    return _lib.lib().pqkv_decode_workspace_bytes(B, Hq, Hkv, S, d)


def test_decode_graph_replays_match_eager():
    """A captured decode call (query rotation, split kernel, merge) replayed
    several times, with eager work and synchronisations in between: every
    replay equals the eager result."""
    B, Hq, Hkv, S, d = 2, 16, 4, 2500, 128
    q, R, Rt, kc, vc, _ = _setup(B, Hq, Hkv, S, d, 4, 4, seed=99)
    qt = torch.from_numpy(q).to(DEV)
    ws = torch.zeros(_lib_decode_bytes((B, Hq, Hkv, S, d)), dtype=torch.uint8, device=DEV)
    eager = attention.decode_attention(qt, kc, vc, Rt, out_dtype=torch.float32, workspace=ws)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):   # warm-up on the capture stream
        attention.decode_attention(qt, kc, vc, Rt, out_dtype=torch.float32, workspace=ws)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        captured = attention.decode_attention(qt, kc, vc, Rt, out_dtype=torch.float32, workspace=ws)
    for i in range(4):
        captured.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager), f"replay {i}"
        attention.decode_attention(qt, kc, vc, Rt, out_dtype=torch.float32, workspace=ws)   # eager call between
        torch.cuda.synchronize()
    _check(eager.cpu().numpy(), _oracle(q, R, kc, vc, S))
