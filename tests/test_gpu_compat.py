"""The reference-compatible exports (polarquant_*_c, the surface llama.cpp
binds with dlsym) and the polarquant_turboquant module, on the GPU."""

import ctypes
import math

import numpy as np
import pytest
import torch

import oracle as OC
from oracle import oracle as O
from polarquant_kv import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _stream():
    return torch.cuda.current_stream().cuda_stream


@pytest.mark.parametrize("d,n_levels", [(128, 16), (128, 8), (64, 16), (128, 4)])
def test_compress_soa_bit_exact(d, n_levels):
    rng = np.random.default_rng(d + n_levels)
    x = (rng.standard_normal((777, d)) * rng.lognormal(0, 1, (777, 1))).astype(np.float32)
    x[0] = 0
    bits = {16: 4, 8: 3, 4: 2}[n_levels]
    cb = O.lloyd_max_codebook(d, bits)[0]
    R = O.rotation_matrix(d, 42).astype(np.float32)
    xt, Rt, cbt = (torch.from_numpy(a).to(DEV) for a in (x, R, cb))
    radius = torch.empty(777, device=DEV)
    packed = torch.empty(777, d // 2, dtype=torch.uint8, device=DEV)
    _lib.lib().polarquant_compress_cuda_c(xt.data_ptr(), Rt.data_ptr(), cbt.data_ptr(), radius.data_ptr(),
                                          packed.data_ptr(), 777, d, n_levels, _stream())
    torch.cuda.synchronize()
    y = OC.c_rotate_fma(x, R)
    r_ref, idx = OC.c_quantize_rotated(y, cb)
    assert np.array_equal(radius.cpu().numpy().view(np.uint32), r_ref.view(np.uint32))
    assert np.array_equal(packed.cpu().numpy(), (idx[:, 0::2] | (idx[:, 1::2] << 4)).astype(np.uint8))


def test_rotate_query_and_inverse_bit_exact():
    d = 128
    x = np.random.default_rng(0).standard_normal((64, d)).astype(np.float32)
    R = O.rotation_matrix(d, 42).astype(np.float32)
    xt, Rt = torch.from_numpy(x).to(DEV), torch.from_numpy(R).to(DEV)
    y = torch.empty_like(xt)
    z = torch.empty_like(xt)
    _lib.lib().polarquant_rotate_query_cuda_c(xt.data_ptr(), Rt.data_ptr(), y.data_ptr(), 64, d, _stream())
    _lib.lib().polarquant_inverse_rotate_cuda_c(y.data_ptr(), Rt.data_ptr(), z.data_ptr(), 64, d, _stream())
    yr = OC.c_rotate_fma(x, R)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), yr.view(np.uint32))
    assert np.array_equal(z.cpu().numpy().view(np.uint32), OC.c_rotate_fma(yr, R, inverse=True).view(np.uint32))


FUSED_CASES = [
    # Hq, Hkv, S, d, n_levels, data
    (8, 2, 300, 128, 16, "channel"),     # outlier channels: radii spread over decades
    (32, 8, 1500, 128, 16, "channel"),   # 8B shape, several splits
    (14, 2, 512, 64, 16, "normal"),      # config-1 shape
    (32, 2, 200, 128, 8, "normal"),      # G = 16, the 3-bit ggml codebook
    (4, 1, 77, 128, 16, "huge"),         # radii past the fp16 range stay exact
]


@pytest.mark.parametrize("case", FUSED_CASES, ids=lambda c: "Hq{}_Hkv{}_S{}_d{}_L{}_{}".format(*c))
def test_fused_attention_soa_matches_oracle(case):
    """polarquant_fused_attention_cuda_c attends with the caller's fp32 radii
    (no fp16 rounding): checked against the SoA oracle fed the same
    unrounded radii, on data whose radii fp16 would change."""
    Hq, Hkv, S, d, n_levels, kind = case
    print(f"compat fused attention {case}", flush=True)
    rng = np.random.default_rng(Hq + S)
    bits = {16: 4, 8: 3}[n_levels]
    import json
    from conftest import GOLDEN
    cb = np.asarray(json.load(open(f"{GOLDEN}/ggml_codebooks.json"))["codebooks"][str(bits)], np.float32)
    if kind == "huge":
        k = (rng.standard_normal((Hkv * S, d)) * 8e3).astype(np.float32)
        v = (rng.standard_normal((Hkv * S, d)) * 8e3).astype(np.float32)
        q_scale = 1e-4
    else:
        src = O.synth_kv(1, Hkv, 2 * S, d, Hq + S, "channel" if kind == "channel" else "normal").astype(np.float32)
        k = src[0, :, :S].reshape(-1, d)
        v = src[0, :, S:].reshape(-1, d)
        q_scale = 1.0
    kr, ki = OC.c_quantize_rotated(k, cb)
    vr, vi = OC.c_quantize_rotated(v, cb)
    assert (kr.astype(np.float16).astype(np.float32) != kr).any()   # fp16 would round these radii
    if kind == "huge":
        assert kr.max() > 65504
    pk, pv = O.pack_codes(ki, 4), O.pack_codes(vi, 4)
    q_rot = (q_scale * rng.standard_normal((Hq, d))).astype(np.float32)
    t = {n: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
         for n, a in dict(q=q_rot, pk=pk, kr=kr, pv=pv, vr=vr, cb=cb).items()}
    out = torch.full((Hq, d), float("nan"), device=DEV)
    scale = 1 / math.sqrt(d)
    _lib.lib().polarquant_fused_attention_cuda_c(t["q"].data_ptr(), t["pk"].data_ptr(), t["kr"].data_ptr(),
                                                 t["pv"].data_ptr(), t["vr"].data_ptr(), t["cb"].data_ptr(),
                                                 out.data_ptr(), Hq, Hkv, S, d, n_levels, ctypes.c_float(scale),
                                                 _stream())
    torch.cuda.synchronize()
    ref = O.decode_attention_soa(q_rot, pk, kr, pv, vr, cb, Hkv, scale)
    got = out.cpu().numpy().astype(np.float64)
    tol = 2e-3 * max(1.0, np.abs(ref).max() / 100)        # relative beyond |o| = 100
    assert np.abs(got - ref).max() <= tol, np.abs(got - ref).max()
    assert (got * ref).sum() / np.linalg.norm(got) / np.linalg.norm(ref) >= 0.9999


def test_init_and_free():
    L = _lib.lib()
    st = L.polarquant_init_c(128, 8, 32, 2, 1024, 4)
    assert st

    class Layer(ctypes.Structure):
        _fields_ = [("k_packed", ctypes.c_void_p), ("k_radius", ctypes.c_void_p),
                    ("v_packed", ctypes.c_void_p), ("v_radius", ctypes.c_void_p)]

    class State(ctypes.Structure):
        _fields_ = [(n, ctypes.c_int) for n in ("enabled", "n_bits", "n_levels", "head_dim", "n_kv_heads",
                                                "n_q_heads", "n_layers", "n_kv_max")] + [
            ("codebook", ctypes.c_void_p), ("rotation", ctypes.c_void_p), ("layers", ctypes.POINTER(Layer))]

    s = ctypes.cast(st, ctypes.POINTER(State)).contents
    assert (s.enabled, s.n_bits, s.n_levels, s.head_dim, s.n_layers) == (1, 4, 16, 128, 2)
    R = np.zeros((128, 128), np.float32)
    torch.cuda.synchronize()
    import ctypes as C
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemcpy(C.c_void_p(R.ctypes.data), C.c_void_p(s.rotation), C.c_size_t(R.nbytes), 2)
    np.testing.assert_allclose(R @ R.T, np.eye(128), atol=1e-4)
    assert s.layers[1].v_radius
    L.polarquant_free_c(st)

    # the codebook is the reference's table for the width (patch:600-613,
    # 978-994); an unsupported width falls back to 4 bits
    import json
    from conftest import GOLDEN
    books = json.load(open(f"{GOLDEN}/ggml_codebooks.json"))["codebooks"]
    for n_bits, want_bits in ((4, 4), (3, 3), (2, 2), (5, 4)):
        st = L.polarquant_init_c(64 if n_bits == 3 else 128, 2, 4, 1, 64, n_bits)
        s = ctypes.cast(st, ctypes.POINTER(State)).contents
        assert (s.n_bits, s.n_levels) == (want_bits, 1 << want_bits)
        cb = np.zeros(s.n_levels, np.float32)
        hip.hipMemcpy(C.c_void_p(cb.ctypes.data), C.c_void_p(s.codebook), C.c_size_t(cb.nbytes), 2)
        assert np.array_equal(cb, np.asarray(books[str(want_bits)], np.float32))
        L.polarquant_free_c(st)


def _soa_codebook(d, kind):
    cb = O.lloyd_max_codebook(d, 4)[0].astype(np.float32)
    rng = np.random.default_rng(11)
    if kind == "unsorted":                   # not increasing: the scan
        return cb[rng.permutation(16)]
    if kind == "repeated":                   # two equal centroids: the scan
        cb = cb.copy()
        cb[9] = cb[8]
        return cb
    if kind == "wide":                       # switch points beyond +-1: the scan
        return np.linspace(-3, 3, 16).astype(np.float32)
    if kind == "random":                     # arbitrary switch points: the table
        return np.sort(rng.uniform(-0.4, 0.4, 16)).astype(np.float32)
    return cb


@pytest.mark.parametrize("kind", ["lloyd", "unsorted", "repeated", "wide", "random"])
@pytest.mark.parametrize("d", [128, 64])
def test_compress_soa_codebooks_and_radii(d, kind):
    """The SoA encoder's quantiser on codebooks that its switch-point table
    refuses (falling back to the scan) or accepts, over radii from zero to
    infinite: the reference's first-minimum scan of the division, bit for
    bit."""
    print(f"compress_soa d={d} codebook={kind}", flush=True)
    rng = np.random.default_rng(d)
    scales = [0.0, 1e-25, 1e-20, 1e-14, 2.0 ** -40 / np.sqrt(d), 1e-12, 1.0, 1e18, 1e20]
    x = np.concatenate([rng.standard_normal((20, d)) * s for s in scales]
                       + [rng.standard_normal((300, d)) * rng.lognormal(0, 1, (300, 1))]).astype(np.float32)
    x[-1, 3] = np.inf
    n = x.shape[0]
    cb = _soa_codebook(d, kind)
    R = O.rotation_matrix(d, 42).astype(np.float32)
    xt, Rt, cbt = (torch.from_numpy(a).to(DEV) for a in (x, R, cb))
    radius = torch.empty(n, device=DEV)
    packed = torch.empty(n, d // 2, dtype=torch.uint8, device=DEV)
    _lib.lib().polarquant_compress_cuda_c(xt.data_ptr(), Rt.data_ptr(), cbt.data_ptr(), radius.data_ptr(),
                                          packed.data_ptr(), n, d, 16, _stream())
    torch.cuda.synchronize()
    r_ref, idx = OC.c_quantize_rotated(OC.c_rotate_fma(x, R), cb)
    assert np.array_equal(radius.cpu().numpy().view(np.uint32), r_ref.view(np.uint32))
    assert np.array_equal(packed.cpu().numpy(), (idx[:, 0::2] | (idx[:, 1::2] << 4)).astype(np.uint8))


@pytest.mark.parametrize("case", ["many_steps", "misaligned"])
def test_compress_soa_long_and_misaligned_inputs(case):
    """The SoA encoder over enough vectors that each workgroup of the
    register-blocked kernel takes several steps (a partial last one), and on
    input 4 bytes off a 16-byte boundary (the four-chain kernel)."""
    print(f"compress_soa {case}", flush=True)
    d = 128
    n = 256 * 128 * 2 + 77 if case == "many_steps" else 999
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((n, d)) * rng.lognormal(0, 1, (n, 1))).astype(np.float32)
    cb = O.lloyd_max_codebook(d, 4)[0].astype(np.float32)
    R = O.rotation_matrix(d, 42).astype(np.float32)
    buf = torch.zeros(n * d + 1, dtype=torch.float32, device=DEV)
    xt = buf[1:] if case == "misaligned" else buf[:-1]
    xt.copy_(torch.from_numpy(x).flatten())
    assert (xt.data_ptr() % 16 == 4) == (case == "misaligned")
    Rt, cbt = torch.from_numpy(R).to(DEV), torch.from_numpy(cb).to(DEV)
    radius = torch.empty(n, device=DEV)
    packed = torch.empty(n, d // 2, dtype=torch.uint8, device=DEV)
    _lib.lib().polarquant_compress_cuda_c(xt.data_ptr(), Rt.data_ptr(), cbt.data_ptr(), radius.data_ptr(),
                                          packed.data_ptr(), n, d, 16, _stream())
    torch.cuda.synchronize()
    r_ref, idx = OC.c_quantize_rotated(OC.c_rotate_fma(x, R), cb)
    assert np.array_equal(radius.cpu().numpy().view(np.uint32), r_ref.view(np.uint32))
    assert np.array_equal(packed.cpu().numpy(), (idx[:, 0::2] | (idx[:, 1::2] << 4)).astype(np.uint8))


# ---- the raw-pointer binding (polarquant_turboquant, flash_turboquant.cu:180-230) ----

@pytest.mark.parametrize("d", [128, 64])
def test_turboquant_compress_bit_exact(d):
    import polarquant_turboquant as tq
    print(f"turboquant_compress d={d}", flush=True)
    N = 1000
    rng = np.random.default_rng(d)
    x = (rng.standard_normal((N, d)) * rng.lognormal(0, 1, (N, 1))).astype(np.float32)
    cb = O.lloyd_max_codebook(d, 4)[0]
    R = O.rotation_matrix(d, 42).astype(np.float32)
    xt, Rt, cbt = (torch.from_numpy(a).to(DEV) for a in (x, R, cb))
    r = torch.zeros(N, device=DEV)
    p = torch.zeros(N, d // 2, dtype=torch.uint8, device=DEV)
    tq.turboquant_compress(xt.data_ptr(), Rt.data_ptr(), cbt.data_ptr(), r.data_ptr(), p.data_ptr(), N, d, 16)
    torch.cuda.synchronize()
    r_ref, idx = OC.c_quantize_rotated(OC.c_rotate_fma(x, R), cb)
    assert np.array_equal(r.cpu().numpy().view(np.uint32), r_ref.view(np.uint32))
    assert np.array_equal(p.cpu().numpy(), O.pack_codes(idx, 4))


TQ_CASES = [
    # Hq, Hkv, S, d, value codebook
    (32, 32, 1024, 128, "same"),      # the reference benchmark's MHA layout (Hq == Hkv)
    (32, 8, 300, 128, "copy"),        # GQA; equal values in a separate tensor
    (14, 2, 40, 64, "scaled"),        # S so small the score buffer cannot hold the plan
]


@pytest.mark.parametrize("case", TQ_CASES, ids=lambda c: "Hq{}_Hkv{}_S{}_d{}_{}".format(*c))
def test_turboquant_full_attention(case):
    """The benchmark's flow (scripts/benchmark_turboquant.py:78-114): fp32
    K/V compressed with turboquant_compress, q_rot = q R^T, attention into
    attn_out (rotated), compared with the SoA oracle on the same bytes, then
    rotated back and compared with attention on the original K/V."""
    import polarquant_turboquant as tq
    Hq, Hkv, S, d, vcb_kind = case
    print(f"turboquant_full_attention {case}", flush=True)
    g = torch.Generator(device=DEV)
    g.manual_seed(S + Hq)
    K = torch.randn(Hkv, S, d, generator=g, device=DEV)
    V = torch.randn(Hkv, S, d, generator=g, device=DEV)
    Q = torch.randn(Hq, d, generator=g, device=DEV)
    R64 = O.rotation_matrix(d, 42)
    R = torch.from_numpy(R64.astype(np.float32)).to(DEV)
    cb = O.lloyd_max_codebook(d, 4)[0]
    k_cb = torch.from_numpy(cb).to(DEV)
    v_cb_np = {"same": cb, "copy": cb.copy(), "scaled": (cb * np.float32(1.25)).astype(np.float32)}[vcb_kind]
    v_cb = k_cb if vcb_kind == "same" else torch.from_numpy(v_cb_np).to(DEV)
    N = Hkv * S
    kr = torch.zeros(N, device=DEV)
    pk = torch.zeros(N, d // 2, dtype=torch.uint8, device=DEV)
    vr = torch.zeros(N, device=DEV)
    pv = torch.zeros(N, d // 2, dtype=torch.uint8, device=DEV)
    tq.turboquant_compress(K.reshape(-1, d).data_ptr(), R.data_ptr(), k_cb.data_ptr(), kr.data_ptr(), pk.data_ptr(),
                           N, d, 16)
    tq.turboquant_compress(V.reshape(-1, d).data_ptr(), R.data_ptr(), v_cb.data_ptr(), vr.data_ptr(), pv.data_ptr(),
                           N, d, 16)
    q_rot = (Q @ R.T).contiguous()
    out = torch.full((Hq, d), float("nan"), device=DEV)
    score = torch.full((Hq, S), float("nan"), device=DEV)
    scale = 1 / math.sqrt(d)
    tq.turboquant_full_attention(q_rot.data_ptr(), R.data_ptr(), pk.data_ptr(), kr.data_ptr(), pv.data_ptr(),
                                 vr.data_ptr(), k_cb.data_ptr(), v_cb.data_ptr(), out.data_ptr(), q_rot.data_ptr(),
                                 score.data_ptr(), out.data_ptr(), Hq, Hkv, S, d, 16, scale)
    torch.cuda.synchronize()
    got = out.cpu().numpy().astype(np.float64)
    c = {n: t.cpu().numpy() for n, t in dict(q=q_rot, pk=pk, kr=kr, pv=pv, vr=vr).items()}
    # the oracle with separate key and value codebooks: values through their own table
    ref_k = O.decode_attention_soa(c["q"], c["pk"], c["kr"], c["pv"], c["vr"], cb, Hkv, scale)
    if vcb_kind == "scaled":
        ref = O.decode_attention_soa(c["q"], c["pk"], c["kr"], c["pv"], c["vr"] * np.float32(1.25), cb, Hkv, scale)
        assert np.abs(ref - ref_k).max() > 0.05          # the value codebook matters
    else:
        ref = ref_k
    assert np.abs(got - ref).max() <= 2e-3
    # rotated back, against attention on the uncompressed K/V (the benchmark's check)
    o = got @ R64
    G = Hq // Hkv
    Kn, Vn, Qn = (t.cpu().numpy().astype(np.float64) for t in (K, V, Q))
    full = np.stack([O.sdpa(Qn[h][None], Kn[h // G], Vn[h // G])[0] for h in range(Hq)])
    if vcb_kind != "scaled":
        cos = (o * full).sum() / np.linalg.norm(o) / np.linalg.norm(full)
        assert cos > 0.98, cos


# ---- head dims other than 64 and 128 (the patch's D-generic kernels) ----

@pytest.mark.parametrize("d", [80, 96, 48, 256, 160])
def test_generic_head_dim_compress_and_rotations_bit_exact(d):
    """polarquant_compress_cuda_c, polarquant_rotate_query_cuda_c and
    polarquant_inverse_rotate_cuda_c at head dims the fixed-d kernels are not
    built for (integration/polarquant-kv.patch:193-269,395-437,508-544 take
    any D): codes and fp32 radii equal the oracle's on the FMA-chain rotation
    (the radius tree over 128 slots up to d = 128, 256 above)."""
    print(f"compat generic d={d}", flush=True)
    rng = np.random.default_rng(d)
    n = 301
    x = (rng.standard_normal((n, d)) * rng.lognormal(0, 1, (n, 1))).astype(np.float32)
    x[0] = 0
    cb = np.asarray(O.lloyd_max_codebook(128, 4)[0], np.float32)
    R = O.rotation_matrix(d, 42).astype(np.float32)
    xt, Rt, cbt = (torch.from_numpy(a).to(DEV) for a in (x, R, cb))
    radius = torch.empty(n, device=DEV)
    packed = torch.empty(n, d // 2, dtype=torch.uint8, device=DEV)
    L = _lib.lib()
    L.polarquant_compress_cuda_c(xt.data_ptr(), Rt.data_ptr(), cbt.data_ptr(), radius.data_ptr(), packed.data_ptr(),
                                 n, d, 16, _stream())
    y = torch.empty_like(xt)
    z = torch.empty_like(xt)
    L.polarquant_rotate_query_cuda_c(xt.data_ptr(), Rt.data_ptr(), y.data_ptr(), n, d, _stream())
    L.polarquant_inverse_rotate_cuda_c(y.data_ptr(), Rt.data_ptr(), z.data_ptr(), n, d, _stream())
    torch.cuda.synchronize()
    yr = OC.c_rotate_fma(x, R)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), yr.view(np.uint32))
    assert np.array_equal(z.cpu().numpy().view(np.uint32), OC.c_rotate_fma(yr, R, inverse=True).view(np.uint32))
    r_ref, idx = O.quantize_rotated(yr, cb)
    assert np.array_equal(radius.cpu().numpy().view(np.uint32), r_ref.view(np.uint32))
    assert np.array_equal(packed.cpu().numpy(), (idx[:, 0::2] | (idx[:, 1::2] << 4)).astype(np.uint8))


@pytest.mark.parametrize("case", [(8, 2, 300, 80), (12, 4, 1000, 96), (4, 4, 129, 256), (6, 1, 700, 48)])
def test_generic_head_dim_attention(case):
    """polarquant_fused_attention_cuda_c and turboquant_full_attention at
    head dims 48, 80, 96 and 256 (the group kernel in its codebook mode):
    within 2e-3 of the SoA oracle on the same codes and fp32 radii; and
    polarquant_init_c accepts the head dim."""
    Hq, Hkv, S, d = case
    print(f"compat generic attention {case}", flush=True)
    rng = np.random.default_rng(S + d)
    cb = np.asarray(O.lloyd_max_codebook(128, 4)[0], np.float32)
    R = O.rotation_matrix(d, 42).astype(np.float32)
    k = rng.standard_normal((Hkv * S, d)).astype(np.float32)
    v = rng.standard_normal((Hkv * S, d)).astype(np.float32)
    L = _lib.lib()
    Rt, cbt = torch.from_numpy(R).to(DEV), torch.from_numpy(cb).to(DEV)
    enc = []
    for a in (k, v):
        at = torch.from_numpy(a).to(DEV)
        rad = torch.empty(Hkv * S, device=DEV)
        pk = torch.empty(Hkv * S, d // 2, dtype=torch.uint8, device=DEV)
        L.polarquant_compress_cuda_c(at.data_ptr(), Rt.data_ptr(), cbt.data_ptr(), rad.data_ptr(), pk.data_ptr(),
                                     Hkv * S, d, 16, _stream())
        enc.append((pk, rad))
    (pk, kr), (pv, vr) = enc
    q_rot = torch.from_numpy(rng.standard_normal((Hq, d)).astype(np.float32)).to(DEV)
    scale = 1.0 / math.sqrt(d)
    out1 = torch.full((Hq, d), float("nan"), device=DEV)
    L.polarquant_fused_attention_cuda_c(q_rot.data_ptr(), pk.data_ptr(), kr.data_ptr(), pv.data_ptr(), vr.data_ptr(),
                                        cbt.data_ptr(), out1.data_ptr(), Hq, Hkv, S, d, 16, scale, _stream())
    out2 = torch.full((Hq, d), float("nan"), device=DEV)
    score = torch.zeros(Hq, S, device=DEV)
    L.turboquant_full_attention(0, Rt.data_ptr(), pk.data_ptr(), kr.data_ptr(), pv.data_ptr(), vr.data_ptr(),
                                cbt.data_ptr(), cbt.data_ptr(), 0, q_rot.data_ptr(), score.data_ptr(), out2.data_ptr(),
                                Hq, Hkv, S, d, 16, scale)
    torch.cuda.synchronize()
    want = O.decode_attention_soa(q_rot.cpu().numpy(), pk.cpu().numpy(), kr.cpu().numpy(), pv.cpu().numpy(),
                                  vr.cpu().numpy(), cb, Hkv, scale)
    for got in (out1, out2):
        g = got.cpu().numpy().astype(np.float64)
        assert np.abs(g - want).max() <= 2e-3
        assert (g * want).sum() / np.linalg.norm(g) / np.linalg.norm(want) >= 0.9999
    st = L.polarquant_init_c(d, Hkv, Hq, 2, 64, 4)
    assert st
    L.polarquant_free_c(st)
