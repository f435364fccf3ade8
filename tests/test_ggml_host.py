"""GGML_TYPE_PQ4 on the host: the type's CPU traits against the oracle, the
oracle's flash_attn_ext against torch's float64 attention, and the backend
ops' argument checks (which fail before any HIP call, so they run without a
GPU)."""

import ctypes
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN
from oracle import oracle as O
from polarquant_kv import _lib, ggml


def _table():
    return np.asarray(json.load(open(os.path.join(GOLDEN, "ggml_codebooks.json")))["codebooks"]["4"], np.float32)


def _rows(n, k, seed, law="normal"):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n, k)).astype(np.float32)
    if law == "scaled":
        x *= np.exp(3 * rng.standard_normal((n, 1))).astype(np.float32)
    return x


def test_default_codebook_is_the_ggml_fixture():
    assert np.array_equal(ggml.default_codebook(), _table())


@pytest.mark.parametrize("d", [64, 128])
def test_rotation_is_orthogonal_and_reproducible(d):
    R = ggml.rotation(d)
    np.testing.assert_allclose(R.astype(np.float64) @ R.T, np.eye(d), atol=2e-5)
    assert np.array_equal(R, ggml.rotation(d))


@pytest.mark.parametrize("d,law", [(128, "normal"), (128, "scaled"), (64, "normal"), (64, "scaled")])
def test_cpu_quantize_rows_equal_the_oracle_bytewise(d, law):
    heads = 4
    x = _rows(300, heads * d, d + (law == "scaled"), law)
    x[0] = 0.0                                   # zero heads: radius 0, direction 0
    x[1, :d] = 1e4                               # norm past 65504: the stored radius saturates
    R = ggml.rotation(d)
    got = ggml.quantize_rows(x, d) if d == 128 else ggml.quantize_rows(x, d, R, _table())
    want = O.ggml_pq4_encode_rows(x, d, R, _table())
    assert got.shape == (300, ggml.row_size(heads * d))
    assert np.array_equal(got, want)
    r16 = got[1, :2].view(np.float16)[0]
    assert r16 == np.float16(65504)


def test_identity_rotation_codes_are_the_brute_force_nearest_entries():
    # R = I: the stored codes are argmin_i |x / |x| - c_i| (first minimum),
    # computed here by numpy over the whole distance matrix, and the stored
    # radius is fp16(|x|)
    d = 64
    x = _rows(200, d, 4)
    c = _table()
    y = ggml.quantize_rows(x, d, np.eye(d, dtype=np.float32), c)
    r = np.sqrt(np.sum(x.astype(np.float64) ** 2, 1))
    dirs = (x / r[:, None].astype(np.float32)).astype(np.float32)
    want = np.argmin(np.abs(dirs[:, :, None] - c[None, None, :]), axis=2)
    blocks = y.reshape(200, d // 32, 18)
    codes = blocks[:, :, 2:].reshape(200, -1)
    got = np.empty((200, d), np.int64)
    got[:, 0::2] = codes & 15
    got[:, 1::2] = codes >> 4
    assert (got == want).mean() > 0.9999
    r16 = blocks[:, 0, :2].copy().view(np.float16)[:, 0].astype(np.float64)
    assert np.all(np.abs(r16 - r) <= np.abs(r) * 2.0 ** -11)


@pytest.mark.parametrize("d", [64, 128])
def test_cpu_dequantize_rows_equal_the_oracle_values(d):
    x = _rows(50, 2 * d, 9)
    R = ggml.rotation(d)
    y = ggml.quantize_rows(x, d, R, _table())
    got = ggml.dequantize_rows(y, 2 * d, d, R, _table())
    want = O.ggml_pq4_values(y.reshape(50, 2, -1), d, R, _table()).reshape(50, 2 * d)
    np.testing.assert_allclose(got, want, rtol=0, atol=1e-5 * np.abs(want).max())
    # and the reconstruction is close to x (4-bit PQ on N(0, 1) data; the
    # table is the d = 128 one, coarser for 64-element heads)
    cos = np.sum(got * x, 1) / np.linalg.norm(got, axis=1) / np.linalg.norm(x, axis=1)
    assert cos.min() > (0.98 if d == 128 else 0.95)


def _torch_sdpa(q, k, v, mask, scale):
    """q [ns][n_q][Hq][d], k / v [ns_k][n_kv][Hkv][d] float64, mask [ns_m][n_q][n_kv] or None."""
    import torch
    ns, n_q, Hq, d = q.shape
    G = Hq // k.shape[2]
    out = np.zeros_like(q)
    for s in range(ns):
        kk = torch.from_numpy(k[s if k.shape[0] > 1 else 0]).transpose(0, 1).repeat_interleave(G, 0)
        vv = torch.from_numpy(v[s if v.shape[0] > 1 else 0]).transpose(0, 1).repeat_interleave(G, 0)
        qq = torch.from_numpy(q[s]).transpose(0, 1)                           # [Hq][n_q][d]
        m = None if mask is None else torch.from_numpy(mask[s if mask.shape[0] > 1 else 0])[None]
        o = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, attn_mask=m, scale=scale)
        out[s] = o.transpose(0, 1).numpy()
    return out


@pytest.mark.parametrize("Hq,Hkv,n_q,ns,ns_k,kind", [(4, 4, 1, 1, 1, "none"), (8, 2, 1, 2, 2, "pad"),
                                                     (6, 2, 5, 1, 1, "causal"), (4, 1, 3, 2, 1, "random")])
def test_oracle_flash_attn_ext_is_torch_sdpa(Hq, Hkv, n_q, ns, ns_k, kind):
    rng = np.random.default_rng(Hq * 10 + n_q)
    d, n_kv = 16, 37
    q = rng.standard_normal((ns, n_q, Hq, d))
    k = rng.standard_normal((ns_k, n_kv, Hkv, d))
    v = rng.standard_normal((ns_k, n_kv, Hkv, d))
    mask = None
    if kind == "pad":
        mask = np.zeros((ns, n_q, n_kv))
        mask[0, :, 30:] = -np.inf
        mask[1, :, 11:] = -np.inf
    elif kind == "causal":
        mask = np.where(np.arange(n_kv)[None, :] <= (n_kv - n_q + np.arange(n_q))[:, None], 0.0, -np.inf)[None]
    elif kind == "random":
        mask = -np.abs(rng.standard_normal((1, n_q, n_kv))) * 3
    scale = 0.3
    got = O.ggml_flash_attn_ext(q, k, v, mask, scale)
    np.testing.assert_allclose(got, _torch_sdpa(q, k, v, mask, scale), rtol=0, atol=1e-12)


def test_oracle_flash_attn_ext_all_masked_row_is_zero():
    q = np.ones((1, 2, 2, 8))
    k = np.ones((1, 5, 1, 8))
    v = np.arange(40.0).reshape(1, 5, 1, 8)
    mask = np.zeros((1, 2, 5))
    mask[0, 1] = -np.inf
    out = O.ggml_flash_attn_ext(q, k, v, mask, 1.0)
    assert not out[0, 1].any()
    np.testing.assert_allclose(out[0, 0, 0], v[0, :, 0].mean(0))


# ---------------------------------------------------------------- argument checks (no HIP call)

class _FakeState(ctypes.Structure):
    _fields_ = ggml._StateFields._fields_


def _fake_state(d=128, bits=4):
    st = _FakeState()
    st.enabled, st.n_bits, st.n_levels, st.head_dim = 1, bits, 1 << bits, d
    st.codebook, st.rotation = 0x1000, 0x2000          # never dereferenced: validation fails first
    return st


def _arr4(t, v):
    return t(*v)


def test_cpy_rejects_bad_arguments_before_any_launch():
    L = _lib.lib()
    st = _fake_state()
    ne = _arr4(_lib.c_int64_4, [100, 3, 1, 1])             # 100 is not whole heads of 128
    nb = _arr4(_lib.c_size_4, [4, 400, 1200, 1200])
    nbd = _arr4(_lib.c_size_4, [18, 54, 162, 162])
    assert L.pqkv_ggml_cpy_pq4(ctypes.byref(st), 0x1000, _lib.F32, ne, nb, 0x2000, nbd, None) == _lib.ERR_INVALID
    assert L.pqkv_ggml_cpy_pq4(None, 0x1000, _lib.F32, ne, nb, 0x2000, nbd, None) == _lib.ERR_INVALID
    st3 = _fake_state(bits=3)
    ne = _arr4(_lib.c_int64_4, [128, 3, 1, 1])
    assert L.pqkv_ggml_cpy_pq4(ctypes.byref(st3), 0x1000, _lib.F32, ne, nb, 0x2000, nbd, None) == _lib.ERR_INVALID
    assert L.pqkv_ggml_cpy_pq4(ctypes.byref(st), 0x1000, _lib.BF16, ne, nb, 0x2000, nbd, None) == _lib.ERR_UNSUPPORTED
    nb_bad = _arr4(_lib.c_size_4, [8, 512, 1536, 1536])   # strided elements
    assert L.pqkv_ggml_cpy_pq4(ctypes.byref(st), 0x1000, _lib.F32, ne, nb_bad, 0x2000, nbd, None) == _lib.ERR_UNSUPPORTED


def test_flash_attn_ext_rejects_bad_arguments_before_any_launch():
    L = _lib.lib()
    st = _fake_state()
    d, n_q, Hq, ns, n_kv, Hkv = 128, 1, 8, 1, 64, 2
    qne = _arr4(_lib.c_int64_4, [d, n_q, Hq, ns])
    qnb = _arr4(_lib.c_size_4, [4, 4 * d * Hq, 4 * d, 4 * d * Hq * n_q])
    kne = _arr4(_lib.c_int64_4, [d, n_kv, Hkv, 1])
    knb = _arr4(_lib.c_size_4, [18, 72 * Hkv, 72, 72 * Hkv * n_kv])
    ws = L.pqkv_ggml_flash_attn_ext_pq4_workspace_bytes(ctypes.byref(st), qne, kne)
    assert ws > 0

    def call(**kw):
        a = dict(q=0x1000, qne=qne, qnb=qnb, kne=kne, knb=knb, vne=kne, vnb=knb, mask=None, mne=None, mnb=None,
                 scale=0.1, max_bias=0.0, softcap=0.0, ws=0x4000, wsb=ws)
        a.update(kw)
        return L.pqkv_ggml_flash_attn_ext_pq4(ctypes.byref(st), a["q"], a["qne"], a["qnb"], 0x2000, a["kne"],
                                              a["knb"], 0x3000, a["vne"], a["vnb"], a["mask"], a["mne"], a["mnb"],
                                              a["scale"], a["max_bias"], a["softcap"], 0x5000, a["ws"], a["wsb"],
                                              None)
    assert call(max_bias=8.0) == _lib.ERR_UNSUPPORTED
    assert call(softcap=30.0) == _lib.ERR_UNSUPPORTED
    assert call(scale=float("inf")) == _lib.ERR_INVALID
    assert call(kne=_arr4(_lib.c_int64_4, [64, n_kv, Hkv, 1])) == _lib.ERR_INVALID       # head size
    assert call(kne=_arr4(_lib.c_int64_4, [d, n_kv, 3, 1]), vne=_arr4(_lib.c_int64_4, [d, n_kv, 3, 1])) \
        == _lib.ERR_INVALID                                                               # 8 heads over 3
    assert call(vne=_arr4(_lib.c_int64_4, [d, n_kv + 1, Hkv, 1])) == _lib.ERR_INVALID   # v differs from k
    assert call(knb=_arr4(_lib.c_size_4, [16, 72 * Hkv, 72, 0])) == _lib.ERR_UNSUPPORTED  # not PQ4 blocks
    assert call(qnb=_arr4(_lib.c_size_4, [8, 4 * d * Hq, 4 * d, 0])) == _lib.ERR_UNSUPPORTED
    mne = _arr4(_lib.c_int64_4, [n_kv - 1, 1, 1, 1])                                       # shorter than n_kv
    mnb = _arr4(_lib.c_size_4, [2, 2 * n_kv, 2 * n_kv, 2 * n_kv])
    assert call(mask=0x6000, mne=mne, mnb=mnb) == _lib.ERR_INVALID
    assert call(wsb=ws - 1) == _lib.ERR_WORKSPACE
