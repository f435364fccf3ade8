"""Host-side parts of the polarquant_kv package (no GPU): codebook, rotation,
JL matrix, layout helpers and the refusal of the GPU entry points to run on
CPU tensors."""

import numpy as np
import pytest
import torch

from polarquant_kv import lloyd_max, qjl, rotation, types
from polarquant_kv import _lib


@pytest.mark.parametrize("d,bits", [(64, 2), (64, 4), (128, 2), (128, 3), (128, 4)])
def test_codebook_matches_reference_golden(d, bits, golden_codebooks):
    c, b = lloyd_max.build_lloyd_max_codebook(d, bits)
    gc, gb = golden_codebooks[f"d{d}_b{bits}"]
    assert np.array_equal(c, gc) and np.array_equal(b, gb)
    t = lloyd_max.get_codebook_torch(d, bits, device="cpu")
    assert t.dtype == torch.float32 and np.array_equal(t.numpy(), gc)
    p = lloyd_max.padded_codebook_torch(d, bits, device="cpu")
    assert p.shape == (16,) and np.array_equal(p[: 1 << bits].numpy(), gc)


def test_quantize_with_codebook_first_minimum():
    c = np.array([-1.0, 0.0, 1.0], np.float32)
    v = np.array([-0.5, 0.5, 0.2, -2.0], np.float32)   # exact ties pick the lower index
    assert list(lloyd_max.quantize_with_codebook(v, c)) == [0, 1, 1, 0]
    assert np.array_equal(lloyd_max.dequantize_with_codebook(np.array([2, 0]), c), [1.0, -1.0])


@pytest.mark.parametrize("d", [64, 128])
def test_rotation_matches_reference_golden(d, golden_R):
    R = rotation.generate_rotation_matrix(d, seed=42)
    assert np.array_equal(R, golden_R[d])
    Rt = rotation.generate_rotation_matrix(d, seed=42, device="cpu")
    assert Rt.dtype == torch.float32 and np.array_equal(Rt.numpy(), golden_R[d].astype(np.float32))
    v = np.random.default_rng(0).standard_normal((4, d)).astype(np.float32)
    np.testing.assert_allclose(rotation.inverse_rotate(rotation.rotate(v, R), R), v, atol=1e-5)


def test_rotation_rejects_bad_dimensions():
    # tests/test_rotation.py:87-103 of the reference
    for bad in (0, -3):
        with pytest.raises(ValueError):
            rotation.generate_rotation_matrix(bad)
    with pytest.raises(ValueError):
        rotation.generate_rotation_matrix(2.5)
    assert abs(rotation.generate_rotation_matrix(1, seed=0)[0, 0]) == 1.0


def test_jl_matrix(golden_P):
    assert np.array_equal(qjl.generate_jl_matrix(128, 128, seed=43), golden_P[(128, 128, 43)])
    with pytest.raises(ValueError):
        qjl.generate_jl_matrix(0, 64)
    s = torch.rand(5, 20) > 0.5
    assert torch.equal(qjl.bit_unpack(qjl.bit_pack(s), 20), s)


def test_cache_layout_helpers():
    assert types.vector_bytes(128, 4) == 72 and types.vector_bytes(64, 2) == 20
    with pytest.raises(ValueError):
        types.vector_bytes(100, 4)
    c = types.PQCache(blocks=torch.zeros(2, 10), head_dim=128, n_bits=(4, 2, 4), seq_len=0, max_seq_len=5,
                      codebooks=None)
    assert c.mixed and c.num_heads == 3
    assert c.head_offset(0) == 0 and c.head_offset(1) == 5 * 72 and c.head_offset(2) == 5 * 72 + 5 * 40


def test_caches_of_one_width_share_the_codebook():
    """Key and value caches of one width and head_dim pass the same codebook
    pointer (decode then serves both from one table); other widths do not."""
    from polarquant_kv import quantizer
    a = quantizer.allocate_cache(1, 2, 8, 64, 4, "cpu")
    b = quantizer.allocate_cache(1, 2, 8, 64, 4, "cpu")
    assert a.codebooks is b.codebooks
    assert quantizer.allocate_cache(1, 2, 8, 64, 2, "cpu").codebooks is not a.codebooks
    assert quantizer.allocate_cache(1, 2, 8, 128, 4, "cpu").codebooks is not a.codebooks
    m1 = quantizer.allocate_cache(1, 2, 8, 64, (4, 2), "cpu")
    m2 = quantizer.allocate_cache(1, 2, 8, 64, [4, 2], "cpu")
    assert m1.codebooks is m2.codebooks and m1.codebooks.shape == (2, 16)
    assert torch.equal(m1.codebooks[0], a.codebooks)


def test_gpu_entry_points_refuse_cpu_tensors():
    from polarquant_kv import attention, quantizer
    x = torch.zeros(1, 1, 4, 128)
    R = torch.eye(128)
    with pytest.raises(ValueError, match="no CPU fallback"):
        quantizer.compress_pq(x, R)
    with pytest.raises(ValueError, match="no CPU fallback"):
        rotation.rotate(x, R)
    kc = _cpu_cache(1, 1, 16, 128)
    with pytest.raises(ValueError, match="no CPU fallback"):
        attention.decode_attention(torch.zeros(1, 2, 128), kc, kc, R)
    with pytest.raises(ValueError, match="no CPU fallback"):
        attention.prefill_attention(torch.zeros(1, 2, 3, 128), kc, kc, R, q_start=0)


def test_missing_library_fails_loudly(monkeypatch):
    monkeypatch.setattr(_lib, "LIB_PATH", "/nonexistent/libpqkv_hip.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(ImportError, match="no CPU fallback"):
        _lib.lib()


def _cpu_cache(B, H, S_max, d, bits=4, seq_len=None):
    from polarquant_kv.quantizer import allocate_cache
    c = allocate_cache(B, H, S_max, d, bits, device="cpu")
    c.seq_len = S_max if seq_len is None else seq_len
    return c


@pytest.mark.parametrize("which", ["values_smaller_S_max", "d_mismatch", "batch_too_big", "value_heads",
                                   "seq_len_mismatch", "rotation_shape", "short_blocks"])
@pytest.mark.parametrize("entry", ["decode", "prefill"])
def test_attention_shape_mismatches_raise_before_any_launch(which, entry):
    """Every disagreement between the query, the two caches and R raises
    ValueError on the host (the kernels address the caches with these
    sizes), for decode and for prefill alike."""
    from polarquant_kv import attention
    B, Hq, Hkv, S, d = 2, 8, 2, 64, 128
    k, v = _cpu_cache(B, Hkv, S, d), _cpu_cache(B, Hkv, S, d)
    R = torch.eye(d)
    q = torch.zeros(B, Hq, d) if entry == "decode" else torch.zeros(B, Hq, 4, d)
    if which == "values_smaller_S_max":
        v = _cpu_cache(B, Hkv, S // 2, d, seq_len=S // 2)
    elif which == "d_mismatch":
        q = q[..., :64]
    elif which == "batch_too_big":
        q = torch.cat([q, q])
    elif which == "value_heads":
        v = _cpu_cache(B, 2 * Hkv, S, d)
    elif which == "seq_len_mismatch":
        v.seq_len = S - 1
    elif which == "rotation_shape":
        R = torch.eye(64)
    elif which == "short_blocks":
        k.blocks = k.blocks[:1]
    with pytest.raises(ValueError) as e:
        if entry == "decode":
            attention.decode_attention(q, k, v, R)
        else:
            attention.prefill_attention(q, k, v, R, q_start=0)
    assert "device tensors" not in str(e.value)       # the shape check, not the device check, fired


def test_max_heads_constant_matches_the_library():
    """include/pqkv.h's PQKV_MAX_HEADS is the library's limit for per-head
    widths: that many kv heads pass validation, one more is refused."""
    import re
    from conftest import ROOT
    import os
    m = re.search(r"#define PQKV_MAX_HEADS\s+(\d+)", open(os.path.join(ROOT, "include", "pqkv.h")).read())
    n = int(m.group(1))
    L = _lib.lib()
    FAKE = 0x1000

    def call(hkv, wsb):
        bits = _lib.int_array([4, 2] * (hkv // 2))
        return L.pqkv_decode_attn(FAKE, 1, FAKE, FAKE, FAKE, FAKE, FAKE, 4, 4, bits, bits, None, None, 0,
                                  1, hkv, hkv, 16, 16, 128, 0.088, FAKE, 1, FAKE, wsb, None)
    # a workspace one byte short: validation reaches the workspace check (the
    # last one before any HIP call) only when the head count is accepted
    need = L.pqkv_decode_workspace_bytes(1, n, n, 16, 128)
    assert call(n, need - 1) == _lib.ERR_WORKSPACE
    need2 = L.pqkv_decode_workspace_bytes(1, n + 2, n + 2, 16, 128)
    assert call(n + 2, need2 - 1) == _lib.ERR_UNSUPPORTED


def test_host_qjl_signatures_and_correction():
    """compute_signatures / compute_correction (python/polarquant_kv/qjl.py:25-57):
    signs = (P e >= 0); correction (1/m) sum (2 s - 1)(P q), 0 for a zero
    residual (tests/test_qjl.py:142-154 asserts that case)."""
    d = 64
    P = qjl.generate_jl_matrix(d, d, seed=43)
    rng = np.random.default_rng(2)
    e = rng.standard_normal(d)
    sig = qjl.compute_signatures(e, P)
    assert sig.jl_dim == d and sig.signs.dtype == bool and sig.signs.shape == (d,)
    assert np.array_equal(sig.signs, P @ e >= 0)
    assert abs(sig.residual_norm - np.linalg.norm(e)) < 1e-12
    q = rng.standard_normal(d)
    want = sum((1.0 if s else -1.0) * float(P[i] @ q) for i, s in enumerate(sig.signs)) / d
    assert abs(qjl.compute_correction(q, sig, P) - want) < 1e-12
    zero = qjl.compute_signatures(np.zeros(d, np.float32), P)
    assert zero.signs.all() and zero.residual_norm == 0.0
    assert qjl.compute_correction(np.ones(d), zero, P) == 0.0


def test_inference_config_validation():
    from polarquant_kv.inference import KVCacheManager, PolarQuantConfig
    with pytest.raises(ValueError):
        KVCacheManager(PolarQuantConfig(n_bits=3), 16, 1, 2, 64, device="cpu")
    with pytest.raises(ValueError):
        KVCacheManager(PolarQuantConfig(enable_qjl=True, jl_dim=32), 16, 1, 2, 64, device="cpu")
    m = KVCacheManager(PolarQuantConfig(), 16, 1, 2, 64, device="cpu")
    assert m.seq_len == 0 and m.memory_bytes == 0 and m.compression_ratio == 0.0
    with pytest.raises(ValueError):
        m.append(torch.zeros(1, 3, 4, 64), torch.zeros(1, 3, 4, 64))   # wrong head count


def test_paged_cache_tables_on_the_host():
    """PagedPQCache bookkeeping (no kernel): page groups are added as
    positions need them, table entry (stream, p) is page p's address for
    that stream, widening the table keeps the entries, and adopt() checks
    caller-managed tables."""
    import torch
    from polarquant_kv.types import PagedPQCache, vector_bytes
    cb = torch.zeros(16)
    c = PagedPQCache(2, 3, 64, 4, cb, "cpu", page_tokens=64, jl_dim=64, max_pages=2)
    assert c.capacity == 0 and c.qjl_signs is not None
    c.ensure(1)
    c.ensure(64)
    assert len(c.groups) == 1
    c.ensure(65)
    c.ensure(200)                                   # 4 pages: the table widens from 2 to 4
    assert len(c.groups) == 4 and c.max_pages == 4 and c.capacity == 256
    vb = vector_bytes(64, 4)
    for p, g in enumerate(c.groups):
        assert tuple(g.shape) == (2, 3, 64, vb)
        want = torch.tensor([g.data_ptr() + s * 64 * vb for s in range(6)])
        assert torch.equal(c.table[:, p], want)
        assert torch.equal(c.sign_table[:, p], torch.tensor([c.sign_groups[p].data_ptr() + s * 64 * 8
                                                             for s in range(6)]))
    with pytest.raises(ValueError):
        PagedPQCache(1, 1, 64, 4, cb, "cpu", page_tokens=96)
    a = PagedPQCache(1, 2, 64, 4, cb, "cpu", page_tokens=64)
    with pytest.raises(ValueError):
        a.adopt(torch.zeros(3, 4, dtype=torch.int64), 256, [])          # wrong stream count
    with pytest.raises(ValueError):
        a.adopt(torch.zeros(2, 4, dtype=torch.int64), 300, [])          # more than the table holds
    a.adopt(torch.zeros(2, 4, dtype=torch.int64), 256, [])
    assert a.capacity == 256
    with pytest.raises(ValueError):
        a.ensure(257)
