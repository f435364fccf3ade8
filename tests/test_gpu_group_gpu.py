"""The reference's GPU group format on the GPU: compress_gpu / decompress_gpu
(src/polarquant_kv_cuda/compress_kernel.py:100-189, decompress_kernel.py:10-51)
bit-exact against the oracle on the same fp32 rotation (the FMA chain of the
C restatement), the QJL residual and sketch, the reference tests' round-trip
thresholds, and the fused attention on the format (compressed_attention_gpu,
polarquant_full.full_compressed_attention, polarquant_kv.attention.
compressed_attention) against the oracle's float64 attention on the same
stored fields."""

import math

import numpy as np
import pytest
import torch

import oracle as OC
from oracle import oracle as O
from polarquant_kv import _lib, attention, quantizer
from polarquant_kv_cuda import compress_kernel, decompress_kernel
from polarquant_kv_cuda.attention_kernel import compressed_attention_gpu
from polarquant_kv_cuda.compressor import get_memory_bytes

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def fma_rotate(x, M, inverse=False):
    """The kernels' fp32 rotation: one FMA chain per output in coordinate order."""
    return OC.c_rotate_fma(np.ascontiguousarray(x, np.float32), np.asarray(M, np.float32), inverse)


def _x(n, d, seed, dtype=np.float32):
    """Vectors with per-vector LogNormal(0, 0.5) norms; row 0 is the zero
    vector and (fp32) row 2 has coordinates past the +-65000 clamp, whose
    radius then saturates at 65504."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((n, d)) * np.exp(0.5 * rng.standard_normal((n, 1)))).astype(dtype)
    x[0] = 0
    if dtype == np.float32 and n > 2:
        x[2, :3] = [1e5, -7e4, 66000.0]
    return x


def _raw_compress(x, R, bits, gs, residual=False):
    """pqkv_group_gpu_compress through the C ABI: the stored fields (and the
    residual) as numpy."""
    n, d = x.shape
    xt = torch.from_numpy(x).to(DEV)
    Rt = torch.from_numpy(R.astype(np.float32)).to(DEV)
    ng = -(-d // gs)
    pd = compress_kernel._packed_dim(ng * gs, bits)
    r = torch.empty(n, dtype=torch.float16, device=DEV)
    c = torch.empty(n, pd, dtype=torch.uint8, device=DEV)
    lo = torch.empty(n, ng, dtype=torch.float16, device=DEV)
    sc = torch.empty(n, ng, dtype=torch.float16, device=DEV)
    e = torch.empty(n, d, dtype=torch.float32, device=DEV) if residual else None
    _lib.check(_lib.lib().pqkv_group_gpu_compress(xt.data_ptr(), _lib.dtype_code(xt.dtype), Rt.data_ptr(),
                                                  Rt.t().contiguous().data_ptr(), n, d, bits, gs, r.data_ptr(),
                                                  c.data_ptr(), lo.data_ptr(), sc.data_ptr(), _lib.F16, _lib.ptr(e),
                                                  _lib.stream_of(xt)))
    out = {k: v.cpu().numpy() for k, v in (("radius", r), ("codes", c), ("mins", lo), ("scales", sc))}
    if residual:
        out["residual"] = e.cpu().numpy()
    return out


@pytest.mark.parametrize("d,bits,gs", [(128, 4, 32), (128, 2, 32), (128, 3, 32), (64, 8, 16), (80, 4, 32),
                                       (96, 2, 32), (128, 4, 128), (64, 5, 8)])
def test_compress_bit_exact_on_the_fma_rotation(d, bits, gs):
    print(f"group gpu compress d={d} bits={bits} gs={gs}", flush=True)
    x = _x(300, d, d + bits + gs)
    R = O.rotation_matrix(d, 42)
    got = _raw_compress(x, R, bits, gs, residual=True)
    want = O.gpu_group_compress(x.astype(np.float32), R, bits, gs, P=O.jl_matrix(64, d, 43), rotate_fn=fma_rotate)
    for k in ("radius", "codes", "mins", "scales"):
        assert np.array_equal(got[k].view(np.uint8), want[k].view(np.uint8)), k
    np.testing.assert_array_equal(got["residual"], want["residual"])


def test_sketch_and_compress_gpu_qjl_fields():
    d, m = 128, 64
    x = _x(400, d, 5, np.float16)
    R = O.rotation_matrix(d, 42)
    P = O.jl_matrix(m, d, 43)
    Rt = torch.from_numpy(R.astype(np.float32)).to(DEV)
    c = compress_kernel.compress_gpu(torch.from_numpy(x).to(DEV)[None, None], Rt, 4, 32,
                                     jl_matrix=torch.from_numpy(P.astype(np.float32)).to(DEV))
    want = O.gpu_group_compress(x.astype(np.float32), R, 4, 32, P=P.astype(np.float32), rotate_fn=fma_rotate)
    proj = want["residual"].astype(np.float64) @ P.astype(np.float32).astype(np.float64).T
    got_bits = O.bit_unpack_lsb(c.qjl_signs[0, 0].cpu().numpy(), m)
    clear = np.abs(proj) > 1e-9
    assert np.array_equal(got_bits[clear], (proj >= 0)[clear])
    assert got_bits[0].all() and c.residual_norms[0, 0, 0].item() == 0          # the zero vector
    np.testing.assert_allclose(c.residual_norms[0, 0].float().cpu().numpy(), want["res_norms"].astype(np.float32),
                               rtol=1e-3)
    assert c.seq_len == c.max_seq_len == 400 and c.original_dim == d and c.n_bits == 4
    assert get_memory_bytes(c) == 400 * (2 + 64 + 8 + 8 + 8 + 2)


@pytest.mark.parametrize("d,bits,gs", [(128, 4, 32), (128, 2, 32), (128, 3, 32), (80, 4, 32)])
def test_decompress_bit_exact(d, bits, gs):
    print(f"group gpu decompress d={d} bits={bits}", flush=True)
    x = _x(200, d, 11)
    R = O.rotation_matrix(d, 42)
    Rt = torch.from_numpy(R.astype(np.float32)).to(DEV)
    c = compress_kernel.compress_gpu(torch.from_numpy(x).to(DEV).reshape(2, 2, 50, d), Rt, bits, gs)
    got = decompress_kernel.decompress_gpu(c, Rt)
    assert got.dtype == torch.float16 and got.shape == (2, 2, 50, d)
    f = lambda t: t.reshape(200, -1).cpu().numpy()        # noqa: E731
    want = O.gpu_group_decompress(f(c.radius), f(c.quantized_direction), f(c.group_mins), f(c.group_scales), R, d,
                                  bits, gs, rotate_fn=fma_rotate)
    assert np.array_equal(got.reshape(200, d).cpu().numpy().view(np.uint16), want.view(np.uint16))


def test_reference_round_trip_thresholds_and_empty():
    """tests/cuda/test_compress_decompress.py:23-80 on the device path."""
    d = 128
    R = torch.from_numpy(O.rotation_matrix(d, 42).astype(np.float32)).to(DEV)
    torch.manual_seed(42)
    kv = torch.randn(1, 1, 16, d, dtype=torch.float16, device=DEV)
    for bits, thr in ((4, 0.99), (3, 0.96), (2, 0.88)):
        c = compress_kernel.compress_gpu(kv, R, n_bits=bits, group_size=32)
        kh = decompress_kernel.decompress_gpu(c, R)
        cos = torch.nn.functional.cosine_similarity(kv.reshape(-1, d).float(), kh.reshape(-1, d).float(), dim=1)
        assert cos.mean().item() >= thr
    e = compress_kernel.compress_gpu(kv[:, :, :0], R)
    assert e.seq_len == 0 and decompress_kernel.decompress_gpu(e, R).shape == (1, 1, 0, d)
    for bad in (dict(n_bits=1), dict(n_bits=9), dict(group_size=0), dict(group_size=129)):
        with pytest.raises(ValueError):
            compress_kernel.compress_gpu(kv, R, **{"n_bits": 4, "group_size": 32, **bad})
    # bf16 input is widened, as kv.float() does
    cb = compress_kernel.compress_gpu(kv.bfloat16(), R)
    assert torch.isfinite(decompress_kernel.decompress_gpu(cb, R).float()).all()


def _fields(c, S):
    f = lambda t: t[:, :, :S].cpu().numpy()                 # noqa: E731
    return f(c.radius), f(c.quantized_direction), f(c.group_mins), f(c.group_scales)


def _recon(c, R, d, S):
    """Unrounded float64 reconstruction of the stored fields, [B, H, S, d]."""
    r, codes, lo, sc = _fields(c, S)
    B, H = r.shape[:2]
    y = O.gpu_group_rotated(r.reshape(-1), codes.reshape(B * H * S, -1), lo.reshape(B * H * S, -1),
                            sc.reshape(B * H * S, -1), d, c.n_bits)
    return (y.astype(np.float64) @ R).reshape(B, H, S, d)


def _check(got, want, tol=2e-3):
    got = np.asarray(got, np.float64)
    err = np.abs(got - want).max()
    cos = (got * want).sum() / (np.linalg.norm(got) * np.linalg.norm(want) + 1e-300)
    assert err <= tol and cos >= 0.9999, (err, cos)


CASES = [  # B, Hq, Hkv, Sq, S, d, bits, gs, qjl m
    (1, 1, 1, 1, 16, 128, 4, 32, 64),
    (2, 8, 2, 1, 1000, 128, 4, 32, 0),
    (1, 4, 4, 5, 300, 64, 2, 32, 0),
    (1, 6, 2, 3, 700, 96, 3, 32, 128),
    (2, 32, 8, 1, 5000, 128, 4, 32, 64),
    (1, 12, 1, 1, 333, 80, 4, 16, 32),
    (1, 2, 1, 9, 129, 128, 8, 64, 0),
]


@pytest.mark.parametrize("case", CASES)
def test_group_attention_vs_oracle(case):
    B, Hq, Hkv, Sq, S, d, bits, gs, m = case
    print(f"group attention {case}", flush=True)
    rng = np.random.default_rng(sum(case))
    R = O.rotation_matrix(d, 42)
    Rt = torch.from_numpy(R.astype(np.float32)).to(DEV)
    k = torch.from_numpy((rng.standard_normal((B, Hkv, S, d))).astype(np.float16)).to(DEV)
    v = torch.from_numpy((rng.standard_normal((B, Hkv, S, d))).astype(np.float16)).to(DEV)
    k[:, :, 0] = 0                                 # a zero key: zero residual, no correction
    P = O.jl_matrix(m, d, 43) if m else None
    Pt = None if P is None else torch.from_numpy(P.astype(np.float32)).to(DEV)
    ck = compress_kernel.compress_gpu(k, Rt, bits, gs, jl_matrix=Pt)
    cv = compress_kernel.compress_gpu(v, Rt, bits, gs)
    q = torch.from_numpy(rng.standard_normal((B, Hq, Sq, d)).astype(np.float16)).to(DEV)
    out = compressed_attention_gpu(q, ck, cv, Rt, jl_matrix=Pt)
    assert out.dtype == torch.float16 and out.shape == q.shape
    got = out.float().cpu().numpy()
    signs = None if P is None else ck.qjl_signs.cpu().numpy()
    norms = None if P is None else ck.residual_norms.float().cpu().numpy()
    qn = q.float().cpu().numpy().astype(np.float64)
    exact = O.group_attention(qn, _recon(ck, R, d, S), _recon(cv, R, d, S), signs=signs, res_norms=norms, P=P)
    _check(got, exact)
    # against the reference's own rounding (the fp16 caches decompress_gpu returns)
    kh = decompress_kernel.decompress_gpu(ck, Rt).float().cpu().numpy()
    vh = decompress_kernel.decompress_gpu(cv, Rt).float().cpu().numpy()
    _check(got, O.group_attention(qn, kh, vh, signs=signs, res_norms=norms, P=P))
    if P is not None:
        # QJL off gives the plain attention
        off = compressed_attention_gpu(q, ck, cv, Rt, jl_matrix=Pt, enable_qjl=False).float().cpu().numpy()
        _check(off, O.group_attention(qn, _recon(ck, R, d, S), _recon(cv, R, d, S)))


def test_group_attention_reference_acceptance():
    """tests/cuda/test_attention_kernel.py:23-90: output shape, cosine >= 0.985
    against SDPA with the JL fixture (64 x 128, torch seed 43), QJL off, and
    zeros for an empty cache."""
    d = 128
    R = torch.from_numpy(O.rotation_matrix(d, 42).astype(np.float32)).to(DEV)
    torch.manual_seed(43)
    P = torch.randn(64, d, dtype=torch.float32, device=DEV) / 8.0
    torch.manual_seed(42)
    Q = torch.randn(1, 1, 1, d, dtype=torch.float16, device=DEV)
    torch.manual_seed(42)
    K = torch.randn(1, 1, 32, d, dtype=torch.float16, device=DEV)
    torch.manual_seed(42)
    V = torch.randn(1, 1, 32, d, dtype=torch.float16, device=DEV)
    std = torch.nn.functional.scaled_dot_product_attention(Q.float(), K.float(), V.float()).half()
    ck = compress_kernel.compress_gpu(K, R, n_bits=4, group_size=32, jl_matrix=P)
    cv = compress_kernel.compress_gpu(V, R, n_bits=4, group_size=32)
    for qjl in (True, False):
        out = compressed_attention_gpu(Q, ck, cv, R, jl_matrix=P, enable_qjl=qjl)
        assert out.shape == Q.shape and out.is_cuda
        cos = torch.nn.functional.cosine_similarity(std.flatten().float(), out.flatten().float(), dim=0).item()
        assert cos >= 0.985
    e = compress_kernel.compress_gpu(K[:, :, :0], R)
    assert not compressed_attention_gpu(Q, e, e, R).any()


def test_polarquant_full_compat_matches_the_oracle():
    """polarquant_full.full_compressed_attention (csrc/polarquant_full.cu:142-186):
    fp32 group fields, original-space query and output, raw pointers."""
    import polarquant_full
    Hq, Hkv, S, d, gs = 8, 4, 700, 128, 32
    ng = d // gs
    rng = np.random.default_rng(8)
    R = O.rotation_matrix(d, 42)
    Rt = torch.from_numpy(R.astype(np.float32)).to(DEV)
    ck = compress_kernel.compress_gpu(torch.from_numpy(rng.standard_normal((1, Hkv, S, d)).astype(np.float16)).to(DEV),
                                      Rt)
    cv = compress_kernel.compress_gpu(torch.from_numpy(rng.standard_normal((1, Hkv, S, d)).astype(np.float16)).to(DEV),
                                      Rt)
    f32 = lambda t: t.float().reshape(Hkv, S, -1).contiguous()        # noqa: E731
    pk, km, ks, kr = ck.quantized_direction[0].contiguous(), f32(ck.group_mins), f32(ck.group_scales), f32(ck.radius)
    pv, vm, vs, vr = cv.quantized_direction[0].contiguous(), f32(cv.group_mins), f32(cv.group_scales), f32(cv.radius)
    q = torch.from_numpy(rng.standard_normal((Hq, d)).astype(np.float32)).to(DEV)
    out = torch.zeros(Hq, d, device=DEV)
    q_rot = torch.zeros(Hq, d, device=DEV)
    score = torch.zeros(Hq, S, device=DEV)
    attn = torch.zeros(Hq, d, device=DEV)
    polarquant_full.full_compressed_attention(q.data_ptr(), Rt.data_ptr(), pk.data_ptr(), km.data_ptr(), ks.data_ptr(),
                                              kr.data_ptr(), pv.data_ptr(), vm.data_ptr(), vs.data_ptr(), vr.data_ptr(),
                                              out.data_ptr(), q_rot.data_ptr(), score.data_ptr(), attn.data_ptr(),
                                              Hq, Hkv, S, d, gs, ng, 1.0 / math.sqrt(d))
    torch.cuda.synchronize()
    want = O.group_attention(q.cpu().numpy().astype(np.float64)[None, :, None], _recon(ck, R, d, S),
                             _recon(cv, R, d, S))[0, :, 0]
    _check(out.cpu().numpy(), want)


@pytest.mark.parametrize("qjl", [False, True])
def test_array_api_compressed_attention_group_semantics(qjl):
    """polarquant_kv.attention.compressed_attention in the reference CPU
    function's format (python/polarquant_kv/attention.py:111-163): group
    codes from quantizer.compress (the same encoder), keys decompressed in
    fp64, QJL signs of the original-space residuals, softmax over all keys.
    2-D with return_scores, and 3-D GQA with one and several query tokens."""
    rng = np.random.default_rng(1 + qjl)
    d, S = 64, 200
    R = O.rotation_matrix(d, 42)
    P = O.jl_matrix(64, d, 43) if qjl else None

    def oracle(q, k, v):
        n = k.shape[0] * k.shape[1]
        r, c, lo, sc = quantizer.group_compress_arrays(k.reshape(n, d), R, 4, 32)
        kh = np.stack([O.group_decompress(r[i], c[i], lo[i], sc[i], R, d, 32) for i in range(n)])
        r2, c2, lo2, sc2 = quantizer.group_compress_arrays(v.reshape(n, d), R, 4, 32)
        vh = np.stack([O.group_decompress(r2[i], c2[i], lo2[i], sc2[i], R, d, 32) for i in range(n)])
        signs = norms = None
        if qjl:
            e = (k.reshape(n, d).astype(np.float32) - kh).astype(np.float64)
            signs = O.bit_pack_lsb(e @ P.T >= 0).reshape(k.shape[0], k.shape[1], -1)[None]
            norms = np.linalg.norm(e, axis=1).reshape(k.shape[0], k.shape[1])[None]
        sh = (1,) + k.shape
        return O.group_attention(q[None].astype(np.float64), kh.reshape(sh), vh.reshape(sh), signs=signs,
                                 res_norms=norms, P=P)[0]

    k2 = rng.standard_normal((S, d)).astype(np.float32)
    v2 = rng.standard_normal((S, d)).astype(np.float32)
    k2[3] = 0.0
    q2 = rng.standard_normal((5, d)).astype(np.float32)
    res = attention.compressed_attention(q2, k2, v2, R, jl_matrix=P, return_scores=True)
    out, scores = res["output"], res["scores"]
    assert out.dtype == np.float32 and out.shape == (5, d) and scores.shape == (5, S)
    want = oracle(q2[None], k2[None], v2[None])[0]
    _check(out, want)
    w = np.exp(scores - scores.max(-1, keepdims=True))
    w /= w.sum(-1, keepdims=True)
    n = S
    r2, c2, lo2, sc2 = quantizer.group_compress_arrays(v2, R, 4, 32)
    vh = np.stack([O.group_decompress(r2[i], c2[i], lo2[i], sc2[i], R, d, 32) for i in range(n)])
    np.testing.assert_allclose(w @ vh, want, atol=2e-3)
    k3 = rng.standard_normal((2, S, d)).astype(np.float32)
    v3 = rng.standard_normal((2, S, d)).astype(np.float32)
    for sq in (1, 7):
        q3 = rng.standard_normal((8, sq, d)).astype(np.float32)
        out3 = attention.compressed_attention(q3, k3, v3, R, jl_matrix=P, num_kv_heads=2)
        assert out3.shape == (8, sq, d)
        _check(out3, oracle(q3, k3, v3))
    with pytest.raises(ValueError):
        attention.compressed_attention(q2, k2, v2, R, n_bits=9)
    empty = attention.compressed_attention(q2, k2[:0], v2[:0], R)
    assert empty.shape == (5, d) and not empty.any()


def test_group_inference_manager_and_layer():
    """polarquant_kv_cuda.inference on the group format: appends in pieces
    equal one compress_gpu of the whole sequence, field for field; the layer's
    compressed attention equals compressed_attention_gpu on the manager's
    caches; the small transformer runs with one manager per layer."""
    from polarquant_kv_cuda.inference.attention import CompressedMultiHeadAttention
    from polarquant_kv_cuda.inference.config import PolarQuantConfig
    from polarquant_kv_cuda.inference.kv_cache import KVCacheManager
    from polarquant_kv_cuda.inference.transformer import SimpleTransformer
    torch.manual_seed(0)
    B, H, d, T = 2, 4, 64, 37
    cfg = PolarQuantConfig(n_bits=4, group_size=32)
    mgr = KVCacheManager(cfg, 64, B, H, d, DEV)
    k = torch.randn(B, H, T, d, device=DEV).half()
    v = torch.randn(B, H, T, d, device=DEV).half()
    mgr.append(k[:, :, :30], v[:, :, :30])
    for t in range(30, T):
        mgr.append(k[:, :, t:t + 1], v[:, :, t:t + 1])
    assert mgr.seq_len == T
    ck, cv = mgr.get_kv()
    whole = compress_kernel.compress_gpu(k, mgr.R, 4, 32)
    for a, b in ((ck.radius, whole.radius), (ck.quantized_direction, whole.quantized_direction),
                 (ck.group_mins, whole.group_mins), (ck.group_scales, whole.group_scales)):
        assert torch.equal(a[:, :, :T], b)
    assert mgr.memory_bytes == 2 * B * H * T * (2 + 32 + 4 + 4) and mgr.compression_ratio > 2
    layer = CompressedMultiHeadAttention(cfg, H * d, H).to(DEV)
    m2 = KVCacheManager(cfg, 64, B, H, d, DEV)
    x = torch.randn(B, 5, H * d, device=DEV)
    y = layer(x, m2)
    kk, vv = m2.get_kv()
    q = layer.q_proj(x).reshape(B, 5, H, d).transpose(1, 2).half()
    att = compressed_attention_gpu(q, kk, vv, m2.R)
    want = layer.o_proj(att.transpose(1, 2).reshape(B, 5, -1).float())
    torch.testing.assert_close(y, want)
    mgr.reset()
    assert mgr.seq_len == 0
    model = SimpleTransformer(cfg, 2, H * d, H, 2, vocab_size=50).to(DEV)
    mgrs = model.create_cache_managers(32, 1, DEV)
    ids = torch.randint(0, 50, (1, 6), device=DEV)
    logits = model(ids, mgrs)
    logits2 = model(ids[:, :1], mgrs)
    assert torch.isfinite(logits).all() and torch.isfinite(logits2).all() and mgrs[0].seq_len == 7
