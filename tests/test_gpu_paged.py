"""Paged caches on the GPU: pqkv_encode_paged, pqkv_decode_attn_paged and
pqkv_prefill_attn_paged through PagedPQCache.

Pages are placed at random slots of one pool (page p of a stream is not next
to page p + 1, and streams interleave), written by appends that cross page
boundaries. Checks: the bytes gathered back through the placement equal one
contiguous encode of the same states (the same encoder); decode and
chunked prefill on the pages equal the contiguous-cache kernels bit for bit
(the same arithmetic, other addresses) and the float64 oracle within the
2e-3 / 0.9999 bar."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from polarquant_kv import attention, quantizer
from polarquant_kv.lloyd_max import padded_codebook_torch
from polarquant_kv.qjl import generate_jl_matrix, rotated_jl_matrix
from polarquant_kv.rotation import generate_rotation_matrix
from polarquant_kv.types import PagedPQCache, vector_bytes

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _random_pages(B, H, d, bits, P, n_pages, seed, jl=0, codebooks=None):
    """A PagedPQCache on pages at random slots of one pool (with spare slots
    no table entry names). Returns the cache and the slot of each (stream,
    page)."""
    n = B * H * n_pages
    gen = torch.Generator().manual_seed(seed)
    slots = torch.randperm(n + 5, generator=gen)[:n].view(B * H, n_pages)
    vb = vector_bytes(d, bits)
    pool = torch.full((n + 5, P, vb), 0xA5, dtype=torch.uint8, device=DEV)   # junk where nothing is written
    cb = padded_codebook_torch(d, bits, DEV) if codebooks is None else codebooks
    c = PagedPQCache(B, H, d, bits, cb, DEV, page_tokens=P, jl_dim=jl)
    table = (pool.data_ptr() + slots * (P * vb)).to(DEV)
    sign_table, storage = None, [pool]
    if jl:
        spool = torch.full((n + 5, P, jl // 8), 0x5A, dtype=torch.uint8, device=DEV)
        sign_table = (spool.data_ptr() + slots * (P * (jl // 8))).to(DEV)
        storage.append(spool)
    c.adopt(table, n_pages * P, storage, sign_table)
    return c, slots


def _gather(c, slots, S):
    """The cache's first S positions through the page placement:
    blocks [B, H, S, vb] (and signs)."""
    pool = c._adopted[1][0]
    B, H = c.batch, c.num_heads
    blocks = pool[slots.to(DEV).flatten()].view(B, H, -1, pool.shape[-1])[:, :, :S]
    signs = None
    if c.jl_dim:
        spool = c._adopted[1][1]
        signs = spool[slots.to(DEV).flatten()].view(B, H, -1, spool.shape[-1])[:, :, :S]
    return blocks, signs


def _states(B, H, S, d, seed, kind="normal"):
    return torch.from_numpy(O.synth_kv(B, H, S, d, seed, kind)).to(DEV)


CASES = [
    # B, Hq, Hkv, d, bits, qjl, S, P, cut (first append length)
    (2, 8, 2, 128, 4, False, 1000, 256, 300),
    (1, 32, 8, 128, 4, False, 4200, 512, 4097),
    (3, 14, 2, 64, 4, False, 777, 64, 65),
    (2, 8, 2, 128, 2, False, 900, 128, 128),
    (2, 8, 4, 64, 2, True, 650, 64, 1),
    (1, 12, 4, 128, 4, True, 1300, 256, 700),
    (2, 4, 4, 128, 4, False, 33, 256, 10),        # one partial page
    (1, 8, 1, 64, 4, True, 512, 256, 256),        # exactly two full pages
]


def _id(c):
    return "B{}_Hq{}_Hkv{}_d{}_b{}_{}_S{}_P{}".format(*c[:5], "qjl" if c[5] else "plain", *c[6:8])


@pytest.mark.parametrize("case", CASES, ids=[_id(c) for c in CASES])
def test_paged_encode_decode_prefill(case):
    B, Hq, Hkv, d, bits, qjl, S, P, cut = case
    print(f"paged {_id(case)}", flush=True)
    R = generate_rotation_matrix(d, seed=42, device=DEV)
    jl_rot = None
    if qjl:
        Pm = generate_jl_matrix(d, d, seed=43)
        jl_rot = rotated_jl_matrix(Pm, R.cpu().numpy(), DEV)
    k = _states(B, Hkv, S, d, 1, "channel")
    v = _states(B, Hkv, S, d, 2)
    n_pages = -(-S // P) + 1
    kp, kslots = _random_pages(B, Hkv, d, bits, P, n_pages, 10, jl=d if qjl else 0)
    vp, vslots = _random_pages(B, Hkv, d, bits, P, n_pages, 11)
    for c, x in ((kp, k), (vp, v)):
        quantizer.compress_pq(x[:, :, :cut].contiguous(), R, cache=c, start=0,
                              jl_rot=jl_rot if c is kp else None)
        quantizer.compress_pq(x[:, :, cut:].contiguous(), R, cache=c, jl_rot=jl_rot if c is kp else None)
    assert kp.seq_len == vp.seq_len == S
    kc = quantizer.compress_pq(k, R, bits, jl_rot=jl_rot)
    vc = quantizer.compress_pq(v, R, bits)
    kb, ks = _gather(kp, kslots, S)
    vb_, _ = _gather(vp, vslots, S)
    assert torch.equal(kb, kc.blocks) and torch.equal(vb_, vc.blocks)
    if qjl:
        assert torch.equal(ks, kc.qjl_signs)

    gq = torch.Generator(device=DEV).manual_seed(5)
    q = torch.randn(B, Hq, d, generator=gq, device=DEV).half()
    got = attention.decode_attention(q, kp, vp, R, jl_rot=jl_rot, out_dtype=torch.float32)
    same = attention.decode_attention(q, kc, vc, R, jl_rot=jl_rot, out_dtype=torch.float32)
    assert torch.equal(got, same)
    cb = O.lloyd_max_codebook(d, bits)[0]
    Pn = Pm if qjl else None
    signs = kc.qjl_signs.cpu().numpy() if qjl else None
    ref = O.decode_attention(q.double().cpu().numpy(), kc.blocks.cpu().numpy(), vc.blocks.cpu().numpy(),
                             R.cpu().numpy().astype(np.float64), cb, cb, k_bits=bits, v_bits=bits,
                             qjl_signs=signs, P=Pn)
    g = got.double().cpu().numpy()
    assert np.abs(g - ref).max() <= 2e-3
    assert (g * ref).sum() / (np.linalg.norm(g) * np.linalg.norm(ref)) >= 0.9999

    Sq = min(S, 70)
    qq = torch.randn(B, Hq, Sq, d, generator=gq, device=DEV).half()
    got_p = attention.prefill_attention(qq, kp, vp, R, q_start=S - Sq, causal=True, jl_rot=jl_rot,
                                        out_dtype=torch.float32)
    same_p = attention.prefill_attention(qq, kc, vc, R, q_start=S - Sq, causal=True, jl_rot=jl_rot,
                                         out_dtype=torch.float32)
    assert torch.equal(got_p, same_p)
    ref_p = O.prefill_attention(qq.double().cpu().numpy(), kc.blocks.cpu().numpy(), vc.blocks.cpu().numpy(),
                                R.cpu().numpy().astype(np.float64), cb, cb, q_start=S - Sq, causal=True,
                                k_bits=bits, v_bits=bits, qjl_signs=signs, P=Pn)
    assert np.abs(got_p.double().cpu().numpy() - ref_p).max() <= 2e-3


def test_paged_own_value_codebook():
    """4-bit keys and values whose codebooks are distinct tensors (the
    kernel keeps a second table) on random pages."""
    B, Hq, Hkv, d, S, P = 2, 8, 2, 128, 600, 128
    R = generate_rotation_matrix(d, seed=42, device=DEV)
    cbk = padded_codebook_torch(d, 4, DEV)
    cbv = cbk.clone()
    k, v = _states(B, Hkv, S, d, 3), _states(B, Hkv, S, d, 4)
    kp, _ = _random_pages(B, Hkv, d, 4, P, 5, 20, codebooks=cbk)
    vp, _ = _random_pages(B, Hkv, d, 4, P, 5, 21, codebooks=cbv)
    quantizer.compress_pq(k, R, cache=kp)
    quantizer.compress_pq(v, R, cache=vp)
    kc = quantizer.compress_pq(k, R, 4)
    vc = quantizer.compress_pq(v, R, 4)
    vc.codebooks = cbv
    q = torch.randn(B, Hq, d, device=DEV).half()
    got = attention.decode_attention(q, kp, vp, R, out_dtype=torch.float32)
    assert torch.equal(got, attention.decode_attention(q, kc, vc, R, out_dtype=torch.float32))


def test_page_groups_grow_without_moving_tokens():
    """A PagedPQCache that allocates its own page groups: appends add pages
    as positions need them, earlier pages are never reallocated (their
    addresses stay in the table), and attention equals the contiguous
    cache's."""
    B, Hq, H, d, P = 2, 4, 2, 64, 64
    R = generate_rotation_matrix(d, seed=42, device=DEV)
    kp = quantizer.allocate_paged_cache(B, H, d, 4, DEV, page_tokens=P)
    vp = quantizer.allocate_paged_cache(B, H, d, 4, DEV, page_tokens=P)
    k, v = _states(B, H, 1100, d, 7), _states(B, H, 1100, d, 8)
    q = torch.randn(B, Hq, d, device=DEV).half()
    first_table = None
    pos = 0
    for n in (1, 63, 1, 200, 1, 1, 600, 233):
        quantizer.compress_pq(k[:, :, pos:pos + n].contiguous(), R, cache=kp)
        quantizer.compress_pq(v[:, :, pos:pos + n].contiguous(), R, cache=vp)
        pos += n
        assert kp.capacity == -(-pos // P) * P and len(kp.groups) == -(-pos // P)
        if first_table is None:
            first_table = kp.table[:, 0].clone()
        assert torch.equal(kp.table[:, 0], first_table)
        kc = quantizer.compress_pq(k[:, :, :pos].contiguous(), R, 4)
        vc = quantizer.compress_pq(v[:, :, :pos].contiguous(), R, 4)
        assert torch.equal(kp.to_contiguous().blocks, kc.blocks)
        got = attention.decode_attention(q, kp, vp, R, out_dtype=torch.float32)
        assert torch.equal(got, attention.decode_attention(q, kc, vc, R, out_dtype=torch.float32))
    assert kp.max_pages >= len(kp.groups) == 18


def test_paged_select_batch_reorders_streams():
    """Beam-style reordering gathers every page group along the batch."""
    B, H, d, P = 3, 2, 64, 64
    R = generate_rotation_matrix(d, seed=42, device=DEV)
    kp = quantizer.allocate_paged_cache(B, H, d, 4, DEV, page_tokens=P)
    vp = quantizer.allocate_paged_cache(B, H, d, 4, DEV, page_tokens=P)
    k, v = _states(B, H, 150, d, 9), _states(B, H, 150, d, 10)
    quantizer.compress_pq(k, R, cache=kp)
    quantizer.compress_pq(v, R, cache=vp)
    idx = torch.tensor([2, 0, 0, 1], device=DEV)
    before_k, before_v = kp.to_contiguous().blocks, vp.to_contiguous().blocks
    kp.select_batch(idx)
    vp.select_batch(idx)
    assert torch.equal(kp.to_contiguous().blocks, before_k[idx])
    q = torch.randn(4, 4, d, device=DEV).half()
    kc = quantizer.compress_pq(k.index_select(0, idx).contiguous(), R, 4)
    vc = quantizer.compress_pq(v.index_select(0, idx).contiguous(), R, 4)
    assert torch.equal(attention.decode_attention(q, kp, vp, R), attention.decode_attention(q, kc, vc, R))
    assert torch.equal(vp.to_contiguous().blocks, before_v[idx])
