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
    of the whole sequence; attention over the manager's cache matches the
    oracle (causal prefill, then decode)."""
    print(f"cache manager bits={bits} qjl={qjl}", flush=True)
    B, H, Hq, d, T0, steps = 2, 2, 8, 64, 100, 5
    cfg = PolarQuantConfig(n_bits=bits, enable_qjl=qjl, jl_dim=d)
    m = KVCacheManager(cfg, max_seq_len=128, batch=B, num_heads=H, head_dim=d, device=DEV)
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
    assert torch.equal(kc.blocks[:, :, :T0 + steps], one.blocks)
    if qjl:
        assert torch.equal(kc.qjl_signs[:, :, :T0 + steps], one.qjl_signs)
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


def test_hf_compressed_cache_on_a_tiny_llama():
    """A randomly initialised 2-layer Llama generates with
    CompressedDynamicCache: every layer keeps only PQ4 bytes, hands the
    model their reconstruction, and the logits stay close to the fp16-cache
    run (the compression error, not a different model)."""
    transformers = pytest.importorskip("transformers")
    from polarquant_kv import hf_integration
    cfg = transformers.LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                                   num_attention_heads=4, num_key_value_heads=2, vocab_size=1000,
                                   max_position_embeddings=512)
    torch.manual_seed(0)
    model = transformers.LlamaForCausalLM(cfg).to(DEV).eval()
    ids = torch.randint(0, 1000, (1, 40), device=DEV)
    with torch.no_grad():
        ref = model(ids, past_key_values=transformers.DynamicCache(), use_cache=True).logits
        hf_integration.patch_model(model, n_bits=4)
        cache = hf_integration.create_compressed_cache(model)
        got = model(ids, past_key_values=cache, use_cache=True).logits
        cos = torch.nn.functional.cosine_similarity(got.flatten().float(), ref.flatten().float(), dim=0)
        assert cos > 0.99, cos
        assert cache.get_seq_length() == 40
        layer = cache.layers[0]
        assert layer.keys.numel() == 0                              # no fp16 states kept
        assert cache.get_compressed_memory_bytes() == 2 * 2 * 2 * 40 * 36   # layers x (K,V) x heads x tokens x 36 B
        assert cache.get_standard_memory_bytes() == 2 * 2 * 2 * 40 * 64 * 2
        # the states the model attended on are the cache's reconstruction
        k_seen, _ = layer.update(torch.zeros(1, 2, 0, 64, device=DEV), torch.zeros(1, 2, 0, 64, device=DEV))
        assert torch.equal(k_seen, quantizer.dequantize(layer.kc, layer.R, k_seen.dtype))
        # greedy decode continues on the compressed cache
        nxt = got[:, -1:].argmax(-1)
        for _ in range(4):
            step = model(nxt, past_key_values=cache, use_cache=True).logits
            nxt = step[:, -1:].argmax(-1)
        assert cache.get_seq_length() == 44
