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


def test_fused_attention_soa_matches_oracle():
    Hq, Hkv, S, d = 8, 2, 300, 128
    rng = np.random.default_rng(4)
    cb = O.lloyd_max_codebook(d, 4)[0]
    k = rng.standard_normal((Hkv * S, d)).astype(np.float32)
    v = rng.standard_normal((Hkv * S, d)).astype(np.float32)
    kr, ki = OC.c_quantize_rotated(k, cb)
    vr, vi = OC.c_quantize_rotated(v, cb)
    pk = (ki[:, 0::2] | (ki[:, 1::2] << 4)).astype(np.uint8)
    pv = (vi[:, 0::2] | (vi[:, 1::2] << 4)).astype(np.uint8)
    q_rot = rng.standard_normal((Hq, d)).astype(np.float32)
    t = {n: torch.from_numpy(a).to(DEV) for n, a in dict(q=q_rot, pk=pk, kr=kr, pv=pv, vr=vr, cb=cb).items()}
    out = torch.empty(Hq, d, device=DEV)
    scale = 1 / math.sqrt(d)
    _lib.lib().polarquant_fused_attention_cuda_c(t["q"].data_ptr(), t["pk"].data_ptr(), t["kr"].data_ptr(),
                                                 t["pv"].data_ptr(), t["vr"].data_ptr(), t["cb"].data_ptr(),
                                                 out.data_ptr(), Hq, Hkv, S, d, 16, ctypes.c_float(scale),
                                                 _stream())
    torch.cuda.synchronize()
    # oracle in the rotated space: identity rotation, fp16-rounded radii as stored in block_pq4
    kb = O.pack_blocks(kr, ki, 4).reshape(1, Hkv, S, -1)
    vb = O.pack_blocks(vr, vi, 4).reshape(1, Hkv, S, -1)
    ref = O.decode_attention(q_rot[None].astype(np.float64), kb, vb, np.eye(d), cb, cb)[0]
    got = out.cpu().numpy()
    assert np.abs(got - ref).max() <= 2e-3
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
    cb = np.zeros(16, np.float32)
    R = np.zeros((128, 128), np.float32)
    torch.cuda.synchronize()
    import ctypes as C
    hip = C.CDLL("libamdhip64.so")
    hip.hipMemcpy(C.c_void_p(cb.ctypes.data), C.c_void_p(s.codebook), C.c_size_t(64), 2)
    hip.hipMemcpy(C.c_void_p(R.ctypes.data), C.c_void_p(s.rotation), C.c_size_t(R.nbytes), 2)
    assert np.array_equal(cb, O.lloyd_max_codebook(128, 4)[0])
    np.testing.assert_allclose(R @ R.T, np.eye(128), atol=1e-4)
    assert s.layers[1].v_radius
    L.polarquant_free_c(st)
