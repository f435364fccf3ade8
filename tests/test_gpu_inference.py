"""The inference cache (polarquant_kv.inference, the reference's
src/polarquant_kv_cuda/inference/) and the Hugging Face cache
(polarquant_kv.hf_integration) on the GPU."""

import math

import numpy as np
import pytest
import torch

from oracle import oracle as O
from polarquant_kv import quantizer
from polarquant_kv.inference import CompressedMultiHeadAttention, KVCacheManager, PolarQuantConfig

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _oracle_prefill(q, kc, vc, R, S, q_start, P=None):
    # (paged caches are gathered into one array first)
    kc = kc.to_contiguous(S) if hasattr(kc, "to_contiguous") else kc
    vc = vc.to_contiguous(S) if hasattr(vc, "to_contiguous") else vc
    d = kc.head_dim
    cb = O.lloyd_max_codebook(d, kc.n_bits)[0]
    signs = None if P is None else kc.qjl_signs.cpu().numpy()[:, :, :S]
    return O.prefill_attention(q.float().cpu().numpy().astype(np.float64), kc.blocks.cpu().numpy()[:, :, :S],
                               vc.blocks.cpu().numpy()[:, :, :S], R.cpu().numpy().astype(np.float64), cb, cb,
                               q_start=q_start, causal=True, k_bits=kc.n_bits, v_bits=vc.n_bits,
                               qjl_signs=signs, P=P)


@pytest.mark.parametrize("bits,qjl", [(4, False), (2, False), (4, True)])
def test_cache_manager_in_place_appends(bits, qjl):
    """Prefill then single-token appends write the same bytes as one encode
    of the whole sequence; attention over the manager's paged cache matches
    the oracle (causal prefill, then decode), across a page boundary."""
    print(f"cache manager bits={bits} qjl={qjl}", flush=True)
    B, H, Hq, d, T0, steps = 2, 2, 8, 64, 100, 5
    cfg = PolarQuantConfig(n_bits=bits, enable_qjl=qjl, jl_dim=d)
    m = KVCacheManager(cfg, max_seq_len=128, batch=B, num_heads=H, head_dim=d, device=DEV, page_tokens=64)
    g = torch.Generator(device=DEV)
    g.manual_seed(0)
    k = torch.randn(B, H, T0 + steps, d, generator=g, device=DEV).half()
    v = torch.randn(B, H, T0 + steps, d, generator=g, device=DEV).half()
    q = torch.randn(B, Hq, T0 + steps, d, generator=g, device=DEV).half()
    m.append(k[:, :, :T0], v[:, :, :T0])
    out0 = m.attend(q[:, :, :T0])
    P = m.jl_matrix if qjl else None
    kc, vc = m.get_kv()
    ref0 = _oracle_prefill(q[:, :, :T0], kc, vc, m.R, T0, 0, P)
    assert np.abs(out0.float().cpu().numpy() - ref0).max() <= 2e-3
    for t in range(T0, T0 + steps):
        m.append(k[:, :, t:t + 1], v[:, :, t:t + 1])
        out = m.attend(q[:, :, t:t + 1])
        ref = _oracle_prefill(q[:, :, t:t + 1], kc, vc, m.R, t + 1, t, P)
        assert np.abs(out.float().cpu().numpy() - ref).max() <= 2e-3
    assert m.seq_len == T0 + steps
    one = quantizer.compress_pq(k, m.R, bits, jl_rot=m.jl_rot)
    flat = kc.to_contiguous()
    assert torch.equal(flat.blocks, one.blocks)
    if qjl:
        assert torch.equal(flat.qjl_signs, one.qjl_signs)
    assert len(kc.groups) == 2 and kc.capacity == 128          # two 64-token pages, no more
    from polarquant_kv.types import vector_bytes
    per = 2 * vector_bytes(d, bits) + (d // 8 if qjl else 0)
    assert m.memory_bytes == B * H * (T0 + steps) * per
    assert abs(m.compression_ratio - (2 * d * 2) / per) < 1e-9
    with pytest.raises(RuntimeError):
        m.append(torch.zeros(B, H, 30, d, device=DEV).half(), torch.zeros(B, H, 30, d, device=DEV).half())
    m.reset()
    assert m.seq_len == 0 and m.memory_bytes == 0


def test_uncompressed_manager_is_plain_attention():
    B, H, d, T = 1, 2, 64, 40
    m = KVCacheManager(PolarQuantConfig(enable_compression=False), 64, B, H, d, device=DEV)
    k = torch.randn(B, H, T, d, device=DEV).half()
    v = torch.randn(B, H, T, d, device=DEV).half()
    q = torch.randn(B, 4, T, d, device=DEV).half()
    m.append(k, v)
    out = m.attend(q).float()
    kk, vv = k.float().repeat_interleave(2, 1), v.float().repeat_interleave(2, 1)
    s = torch.matmul(q.float(), kk.transpose(-1, -2).contiguous()) / math.sqrt(d)
    s = s.masked_fill(torch.ones(T, T, dtype=torch.bool, device=DEV).triu(1), float("-inf"))
    ref = torch.matmul(torch.softmax(s, -1), vv)
    assert (out - ref).abs().max() < 2e-3
    assert m.compression_ratio == 1.0


@torch.no_grad()
def test_compressed_attention_layer_prefill_then_decode():
    torch.manual_seed(0)
    E, Hq, Hkv, d = 256, 4, 2, 64
    layer = CompressedMultiHeadAttention(PolarQuantConfig(n_bits=4), E, Hq, Hkv).to(DEV)
    m = KVCacheManager(PolarQuantConfig(n_bits=4), 64, 1, Hkv, d, device=DEV)
    x = torch.randn(1, 20, E, device=DEV)
    y0 = layer(x[:, :16], m)
    y1 = layer(x[:, 16:17], m)
    assert y0.shape == (1, 16, E) and y1.shape == (1, 1, E) and m.seq_len == 17
    # the layer's attention is the oracle's on the cached bytes
    q = layer.q_proj(x[:, :17]).reshape(1, 17, Hq, d).transpose(1, 2).half()
    kc, vc = m.get_kv()
    ref = _oracle_prefill(q, kc, vc, m.R, 17, 0)
    o = torch.from_numpy(ref).float().to(DEV).transpose(1, 2).reshape(1, 17, -1)
    want = layer.o_proj(o)
    assert (torch.cat([y0, y1], 1) - want).abs().max() < 5e-3


def _tiny_llama(dtype=torch.float32):
    transformers = pytest.importorskip("transformers")
    cfg = transformers.LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, vocab_size=1000,
                                   max_position_embeddings=512)
    torch.manual_seed(0)
    return transformers, transformers.LlamaForCausalLM(cfg).to(DEV, dtype).eval()


@torch.no_grad()
def test_hf_fused_attention_on_a_tiny_llama():
    """A randomly initialised 2-layer Llama patched with patch_model attends
    through the registered polarquant attention: every layer keeps only
    paged PQ4 bytes, the fused decode / prefill kernels run on them (no fp16
    keys or values), the layer's attention equals the oracle's on the cached
    bytes, and the logits equal those of the same model attending (SDPA) on
    the cache's reconstruction."""
    transformers, model = _tiny_llama()
    from polarquant_kv import hf_integration
    ids = torch.randint(0, 1000, (1, 40), device=DEV)
    ref = model(ids, past_key_values=transformers.DynamicCache(), use_cache=True).logits
    # the same compressed representation, read back by SDPA (reconstruction mode)
    recon_cache = hf_integration.CompressedDynamicCache(n_bits=4)
    recon = model(ids, past_key_values=recon_cache, use_cache=True).logits
    hf_integration.patch_model(model, n_bits=4)
    assert model.config._attn_implementation == hf_integration.ATTENTION_NAME
    cache = hf_integration.create_compressed_cache(model)
    assert cache.fused
    got = model(ids, past_key_values=cache, use_cache=True).logits
    cos = torch.nn.functional.cosine_similarity(got.flatten().float(), ref.flatten().float(), dim=0)
    assert cos > 0.99, cos
    assert (got - recon).abs().max() < 1e-3 * recon.abs().max()
    assert cache.get_seq_length() == 40
    layer = cache.layers[0]
    assert layer.keys.numel() == 0 and layer.values.numel() == 0     # no fp16 states kept
    assert cache.get_compressed_memory_bytes() == 2 * 2 * 2 * 40 * 36   # layers x (K,V) x heads x tokens x 36 B
    assert cache.get_standard_memory_bytes() == 2 * 2 * 2 * 40 * 64 * 2
    # the layer's attention is the oracle's on its cached bytes
    q1 = torch.randn(1, 4, 1, 64, device=DEV)
    q8 = torch.randn(1, 4, 8, 64, device=DEV)
    for q in (q1, q8):
        out = layer.attend(q, 64 ** -0.5)
        want = _oracle_prefill(q, layer.kc, layer.vc, layer.R, 40, 40 - q.shape[2])
        assert np.abs(out.double().cpu().numpy() - want).max() <= 2e-3
    # greedy decode continues on the compressed cache, step by step in
    # agreement with the reconstruction path
    nxt = got[:, -1:].argmax(-1)
    for _ in range(4):
        step = model(nxt, past_key_values=cache, use_cache=True).logits
        model.set_attn_implementation("sdpa")
        step_r = model(nxt, past_key_values=recon_cache, use_cache=True).logits
        model.set_attn_implementation(hf_integration.ATTENTION_NAME)
        assert (step - step_r).abs().max() < 1e-3 * step_r.abs().max()
        nxt = step[:, -1:].argmax(-1)
    assert cache.get_seq_length() == 44
    # generate() drives the same path (its masks are None for an unpadded batch)
    gen = model.generate(ids, past_key_values=hf_integration.create_compressed_cache(model), max_new_tokens=6,
                         do_sample=False)
    model.set_attn_implementation("sdpa")
    gen_r = model.generate(ids, past_key_values=hf_integration.CompressedDynamicCache(n_bits=4), max_new_tokens=6,
                           do_sample=False)
    assert torch.equal(gen, gen_r)


@torch.no_grad()
def test_hf_fused_attention_bf16_model():
    """A bf16 model: states are widened to fp32 for the encoder and the
    queries for the kernels; the output goes back to bf16."""
    transformers, model = _tiny_llama(torch.bfloat16)
    from polarquant_kv import hf_integration
    ids = torch.randint(0, 1000, (1, 24), device=DEV)
    ref = model(ids, past_key_values=transformers.DynamicCache(), use_cache=True).logits.float()
    hf_integration.patch_model(model, n_bits=4)
    cache = hf_integration.create_compressed_cache(model)
    got = model(ids, past_key_values=cache, use_cache=True).logits.float()
    assert got.dtype == torch.float32 and torch.isfinite(got).all()
    cos = torch.nn.functional.cosine_similarity(got.flatten(), ref.flatten(), dim=0)
    assert cos > 0.98, cos
    step = model(got[:, -1:].argmax(-1), past_key_values=cache, use_cache=True).logits
    assert torch.isfinite(step.float()).all() and cache.get_seq_length() == 25


@torch.no_grad()
def test_hf_fused_cache_beam_reorder():
    """reorder_cache gathers the pages along the batch: attention after a
    reorder equals attention on caches built from the reordered states."""
    transformers, model = _tiny_llama()
    from polarquant_kv import hf_integration
    hf_integration.patch_model(model, n_bits=4)
    cache = hf_integration.create_compressed_cache(model)
    ids = torch.randint(0, 1000, (3, 20), device=DEV)
    model(ids, past_key_values=cache, use_cache=True)
    beam = torch.tensor([2, 2, 0], device=DEV)
    before = cache.layers[1].kc.to_contiguous().blocks
    cache.reorder_cache(beam)
    assert torch.equal(cache.layers[1].kc.to_contiguous().blocks, before[beam])
    cache2 = hf_integration.create_compressed_cache(model)
    model(ids[beam], past_key_values=cache2, use_cache=True)
    nxt = torch.randint(0, 1000, (3, 1), device=DEV)
    a = model(nxt, past_key_values=cache, use_cache=True).logits
    b = model(nxt, past_key_values=cache2, use_cache=True).logits
    assert torch.equal(a, b)
