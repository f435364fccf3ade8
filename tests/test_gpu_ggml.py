"""GGML_TYPE_PQ4 backend ops on the GPU: cpy against the type's CPU trait
(bytewise), flash_attn_ext against the oracle's float64 attention on the
rows' values, in llama.cpp's cache layout (a token's heads side by side,
permuted views) with padding, causal, random and fully masking masks."""

import json
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import oracle as O
from polarquant_kv import ggml

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _table():
    return np.asarray(json.load(open(os.path.join(GOLDEN, "ggml_codebooks.json")))["codebooks"]["4"], np.float32)


@pytest.mark.parametrize("d,dtype,ns", [(128, torch.float32, 1), (128, torch.float16, 2), (64, torch.float32, 3)])
def test_cpy_writes_the_cpu_traits_bytes_in_place(d, dtype, ns):
    print(f"ggml cpy d={d} {dtype} ns={ns}", flush=True)
    Hkv, n_tok, n_max, p0, pad = 4, 37, 80, 11, 6
    rng = np.random.default_rng(d + ns)
    x = (rng.standard_normal((1, ns, n_tok, Hkv * d)) * np.exp(rng.standard_normal((1, ns, n_tok, 1)))).astype(np.float32)
    x[0, 0, 0] = 0.0
    x[0, 0, 1, :d] = 1e4 if dtype == torch.float32 else 6e3
    src = torch.from_numpy(x).to(DEV, dtype)
    row = ggml.row_size(Hkv * d)
    cache = torch.full((1, ns, n_max, row + pad), 0xAB, dtype=torch.uint8, device=DEV)
    dst = cache[:, :, p0:p0 + n_tok, :row]
    with ggml.State(d, Hkv, Hkv) as st:
        ggml.cpy(st, src, dst)
        torch.cuda.synchronize()
    got = cache.cpu().numpy()
    want = ggml.quantize_rows(src.float().cpu().numpy(), d, ggml.rotation(d), _table())
    assert np.array_equal(got[:, :, p0:p0 + n_tok, :row], want)
    untouched = np.ones(got.shape, bool)
    untouched[:, :, p0:p0 + n_tok, :row] = False
    assert np.all(got[untouched] == 0xAB)


def _case(d, Hq, Hkv, n_q, ns, ns_kv, n_kv, kind, seed):
    """llama.cpp-layout caches filled by the cpy op, a permuted query view,
    the mask; returns the device views and the oracle's inputs."""
    rng = np.random.default_rng(seed)
    vb = ggml.row_size(d)
    n_max = n_kv + 19
    caches, values = [], []
    st = ggml.State(d, Hkv, Hq)
    for _ in range(2):
        x = rng.standard_normal((1, ns_kv, n_kv, Hkv * d)).astype(np.float32)
        cache = torch.zeros((ns_kv, n_max, Hkv * vb), dtype=torch.uint8, device=DEV)
        ggml.cpy(st, torch.from_numpy(x).to(DEV), cache[None, :, :n_kv])
        caches.append(cache)
    torch.cuda.synchronize()
    R = ggml.rotation(d)
    for cache in caches:
        b = cache.cpu().numpy()[:, :n_kv].reshape(ns_kv, n_kv, Hkv, vb)
        values.append(O.ggml_pq4_values(b, d, R, _table()))
    views = [c.view(ns_kv, n_max, Hkv, vb)[:, :n_kv].permute(0, 2, 1, 3) for c in caches]
    q_cur = torch.from_numpy(rng.standard_normal((ns, n_q, Hq, d)).astype(np.float32)).to(DEV)
    q = q_cur.permute(0, 2, 1, 3)                       # [ns][Hq][n_q][d], token stride Hq*d
    mask = None
    m_np = None
    if kind is not None:
        ns_m = ns if kind in ("pad", "rowmasked") else 1
        n_q_pad, n_kv_pad = (n_q + 31) // 32 * 32, n_kv + 5
        m = np.full((ns_m, 1, n_q_pad, n_kv_pad), -np.inf, np.float32)
        if kind == "pad":
            for s in range(ns_m):
                m[s, 0, :, :n_kv - 17 * (s + 1)] = 0.0
        elif kind == "causal":
            for i in range(n_q):
                m[0, 0, i, :n_kv - n_q + i + 1] = 0.0
        elif kind == "random":
            m[0, 0, :, :n_kv] = -np.abs(rng.standard_normal((n_q_pad, n_kv))) * 2
        elif kind == "rowmasked":
            m[:, 0, :, :n_kv] = 0.0
            m[0, 0, n_q - 1, :] = -np.inf               # the last row of sequence 0 sees nothing
        mask = torch.from_numpy(m).to(DEV, torch.float16)
        m_np = mask.float().cpu().numpy()[:, 0, :n_q, :n_kv].astype(np.float64)
    return st, q, views, mask, q_cur.cpu().numpy(), values, m_np


@pytest.mark.parametrize("d,Hq,Hkv,n_q,ns,ns_kv,n_kv,kind", [
    (128, 32, 8, 1, 1, 1, 1000, "pad"),
    (128, 8, 8, 1, 2, 2, 777, None),
    (64, 14, 2, 1, 3, 1, 300, "random"),
    (128, 8, 1, 7, 1, 1, 300, "causal"),
    (128, 28, 4, 1, 1, 1, 500, "pad"),
    (128, 4, 4, 2, 2, 2, 64, "rowmasked"),
    (64, 6, 2, 3, 1, 1, 1, None),
    (128, 32, 8, 1, 1, 1, 16384, "pad"),
    (128, 32, 8, 3, 2, 2, 500, "causal"),   # one kv head per wave, 3 query rows x 2 sequences
    (64, 16, 4, 1, 2, 2, 600, "pad"),       # one kv head per wave at d = 64
    (64, 8, 8, 2, 1, 1, 333, "random"),
])
def test_flash_attn_ext_matches_the_oracle(d, Hq, Hkv, n_q, ns, ns_kv, n_kv, kind):
    print(f"ggml flash_attn_ext d={d} Hq={Hq} Hkv={Hkv} n_q={n_q} ns={ns} ns_kv={ns_kv} n_kv={n_kv} {kind}",
          flush=True)
    st, q, (kv, vv), mask, q_np, (k_val, v_val), m_np = _case(d, Hq, Hkv, n_q, ns, ns_kv, n_kv, kind, n_kv + Hq)
    scale = 1.0 / np.sqrt(d)
    out = ggml.flash_attn_ext(st, q, kv, vv, mask, scale)
    torch.cuda.synchronize()
    st.close()
    want = O.ggml_flash_attn_ext(q_np, k_val, v_val, m_np, scale)
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    err = np.abs(got - want).max()
    assert err <= 2e-3, err
    if kind == "rowmasked":
        assert not got[0, n_q - 1].any()


def test_flash_attn_ext_empty_cache_gives_zeros():
    d, Hq, Hkv = 128, 4, 2
    with ggml.State(d, Hkv, Hq) as st:
        q = torch.randn(1, Hq, 1, d, device=DEV)
        k = torch.zeros((1, Hkv, 0, ggml.row_size(d)), dtype=torch.uint8, device=DEV)
        out = ggml.flash_attn_ext(st, q, k, k, None, 0.1)
        torch.cuda.synchronize()
    assert out.shape == (1, 1, Hq, d) and not out.cpu().any()


def _sweep_shape(seed):
    rng = np.random.default_rng(4000 + seed)
    d = int(rng.choice([64, 128]))
    Hkv = int(rng.choice([1, 2, 4, 8]))
    Hq = Hkv * int(rng.integers(1, 9))
    n_q = int(rng.integers(1, 5))
    ns = int(rng.integers(1, 4))
    ns_kv = int(rng.choice([1, ns]))
    n_kv = int(rng.integers(n_q + 20, 3000))
    kind = [None, "pad", "causal", "random"][int(rng.integers(0, 4))]
    return d, Hq, Hkv, n_q, ns, ns_kv, n_kv, kind


@pytest.mark.parametrize("seed", range(12))
def test_flash_attn_ext_random_shapes(seed):
    """Seeded random shapes (head_dim, GQA group, query rows, sequences that
    share one cache or have their own, cache length, mask kind) against the
    oracle, as test_flash_attn_ext_matches_the_oracle."""
    test_flash_attn_ext_matches_the_oracle(*_sweep_shape(seed))
