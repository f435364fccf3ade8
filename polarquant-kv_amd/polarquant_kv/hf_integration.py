"""Hugging Face transformers integration (transformers 5 cache and attention
APIs).

Mirrors src/polarquant_kv_cuda/hf_integration.py of the reference
(CompressedDynamicCache, patch_model, create_compressed_cache). The
reference's cache keeps the model's fp16 states and adds compressed copies
that nothing reads (hf_integration.py:43-62), so its model still attends on
the original states. Here:

  - each layer keeps only paged PQ caches (block_pq4 / block_pq2,
    PagedPQCache: pages of page_tokens positions added as the sequence
    grows, new states encoded straight into their pages by the HIP encoder;
    the reference's per-layer rotation seeds 42 + layer);
  - patch_model registers an attention function, ATTENTION_NAME, with
    transformers' AttentionInterface (and the flash-style mask function,
    which hands it None unless the batch is padded) and switches the model
    to it. Each layer's attention then runs the fused kernels on the layer's
    caches: decode (pqkv_decode_attn_paged) for one new token, causal
    chunked prefill (pqkv_prefill_attn_paged) for several. update() encodes
    the new states and returns handles of the layer (empty tensors), so no
    fp16 key or value of the cache is ever materialised;
  - a cache whose model uses any other attention implementation (a
    CompressedDynamicCache built without patch_model) hands the model the
    reconstruction r16 c[code] R of the whole cache instead (pqkv_dequantize),
    which that implementation can read.

Padded batches (an attention mask with masked positions) are refused: the
fused kernels apply the causal rule only.
"""

from __future__ import annotations

import torch

from . import attention, quantizer
from .types import PagedPQCache

ATTENTION_NAME = "polarquant"


def _cache_utils():
    try:
        from transformers.cache_utils import DynamicCache, DynamicLayer
    except ImportError as e:            # pragma: no cover - transformers is optional
        raise ImportError("the Hugging Face integration needs transformers >= 5") from e
    return DynamicCache, DynamicLayer


def polarquant_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    """transformers attention function (AttentionInterface signature): query
    [B, Hq, Sq, d] against the compressed caches of the layer whose handles
    `key` / `value` are -> ([B, Sq, Hq, d], None)."""
    layer = getattr(key, "_pq_layer", None)
    if layer is None:
        raise RuntimeError(f"the {ATTENTION_NAME!r} attention reads a CompressedDynamicCache made by "
                           "create_compressed_cache(model) after patch_model(model)")
    if attention_mask is not None:
        raise NotImplementedError("padded batches: the fused PolarQuant kernels apply the causal rule only")
    if dropout:
        raise NotImplementedError("attention dropout")
    return layer.attend(query, scaling).transpose(1, 2).contiguous(), None


def register_attention() -> str:
    """Register ATTENTION_NAME with transformers' attention and mask
    interfaces (idempotent); returns the name."""
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface, flash_attention_mask
    AttentionInterface.register(ATTENTION_NAME, polarquant_attention)
    AttentionMaskInterface.register(ATTENTION_NAME, flash_attention_mask)
    return ATTENTION_NAME


def _layer_class():
    _, DynamicLayer = _cache_utils()

    class CompressedLayer(DynamicLayer):
        """One layer of CompressedDynamicCache: paged key and value caches."""

        def __init__(self, layer_idx: int, n_bits: int, page_tokens: int, fused: bool):
            super().__init__()
            self.layer_idx = layer_idx
            self.n_bits = n_bits
            self.page_tokens = page_tokens
            self.fused = fused
            self.kc: PagedPQCache | None = None
            self.vc: PagedPQCache | None = None
            self.R = None

        def lazy_initialization(self, key_states, value_states, *args, **kwargs):
            from .rotation import generate_rotation_matrix
            self.dtype, self.device = key_states.dtype, key_states.device
            self.R = generate_rotation_matrix(key_states.shape[-1], seed=42 + self.layer_idx, device=self.device)
            # the layer keeps no fp16 states
            self.keys = torch.empty(0, dtype=self.dtype, device=self.device)
            self.values = torch.empty(0, dtype=self.dtype, device=self.device)
            self.is_initialized = True

        def update(self, key_states, value_states, *args, **kwargs):
            if not self.is_initialized:
                self.lazy_initialization(key_states, value_states)
            B, H, T, d = key_states.shape
            if self.kc is None:
                self.kc = quantizer.allocate_paged_cache(B, H, d, self.n_bits, self.device,
                                                         page_tokens=self.page_tokens)
                self.vc = quantizer.allocate_paged_cache(B, H, d, self.n_bits, self.device,
                                                         page_tokens=self.page_tokens)
            start = self.get_seq_length()
            quantizer.compress_pq(key_states, self.R, cache=self.kc, start=start)
            quantizer.compress_pq(value_states, self.R, cache=self.vc, start=start)
            if self.fused:
                # handles for polarquant_attention, no states
                k = key_states.new_empty((B, H, 0, d))
                v = value_states.new_empty((B, H, 0, d))
                k._pq_layer = v._pq_layer = self
                return k, v
            out_dtype = self.dtype if self.dtype in (torch.float16, torch.float32) else torch.float32
            keys = quantizer.dequantize(self.kc, self.R, out_dtype)
            values = quantizer.dequantize(self.vc, self.R, out_dtype)
            return keys.to(self.dtype), values.to(self.dtype)

        def attend(self, query: torch.Tensor, scaling: float | None = None) -> torch.Tensor:
            """query [B, Hq, Sq, d] at the last Sq cached positions ->
            [B, Hq, Sq, d] in the query's dtype: the fused decode kernel for
            Sq = 1, causal chunked prefill otherwise."""
            B, Hq, Sq, d = query.shape
            S = self.get_seq_length()
            if S == 0 or Sq == 0:
                return torch.zeros_like(query)
            q = query if query.dtype in (torch.float16, torch.float32) else query.float()
            if Sq == 1:
                out = attention.decode_attention(q[:, :, 0], self.kc, self.vc, self.R, scale=scaling).unsqueeze(2)
            else:
                out = attention.prefill_attention(q, self.kc, self.vc, self.R, q_start=S - Sq, causal=True,
                                                  scale=scaling)
            return out.to(query.dtype)

        def get_seq_length(self) -> int:
            return 0 if self.kc is None else self.kc.seq_len

        def get_mask_sizes(self, query_length: int, *args, **kwargs):
            return self.get_seq_length() + query_length, 0

        def crop(self, tokens_to_remove: int) -> None:
            """DynamicLayer.crop's rule (transformers 5): a negative value
            removes that many tokens, a positive one is the legacy absolute
            length to keep (nothing happens when it is not below the current
            length), and 0 does nothing. The pages stay allocated."""
            if self.kc is None or tokens_to_remove == 0:
                return
            S = self.kc.seq_len
            if tokens_to_remove > 0:
                if tokens_to_remove >= S:
                    return
                keep = tokens_to_remove
            else:
                keep = max(0, S + tokens_to_remove)
            self.kc.seq_len = self.vc.seq_len = keep

        def reset(self) -> None:
            if self.kc is not None:
                self.kc.seq_len = self.vc.seq_len = 0

        def compressed_bytes(self) -> int:
            """Bytes of the cached positions (K + V)."""
            if self.kc is None:
                return 0
            n = self.kc.batch * self.kc.num_heads * self.kc.seq_len
            from .types import vector_bytes
            return 2 * n * vector_bytes(self.kc.head_dim, self.n_bits)

        def _select(self, index: torch.Tensor) -> None:
            if self.kc is not None:
                self.kc.select_batch(index)
                self.vc.select_batch(index)

        def batch_repeat_interleave(self, repeats: int):
            if self.kc is not None:
                self._select(torch.arange(self.kc.batch, device=self.device).repeat_interleave(repeats))

        def batch_select_indices(self, indices):
            self._select(torch.as_tensor(indices, device=self.device, dtype=torch.int64))

        def reorder_cache(self, beam_idx):
            self._select(beam_idx.to(device=self.device, dtype=torch.int64))

    return CompressedLayer


def CompressedDynamicCache(n_bits: int = 4, group_size: int = 32, head_dim: int | None = None,
                           num_layers: int | None = None, page_tokens: int = 256, fused: bool = False):
    """A transformers DynamicCache whose layers store only the PQ-encoded
    keys and values (hf_integration.py:21 of the reference keeps the same
    constructor arguments; head_dim and num_layers are taken from the states
    as they arrive, and group_size is checked like the reference's). fused:
    the model attends through polarquant_attention (create_compressed_cache
    sets it for a patched model); otherwise the layers hand the model the
    cache's reconstruction."""
    DynamicCache, _ = _cache_utils()
    quantizer._validate_params(n_bits, group_size, head_dim or group_size)
    if n_bits not in (2, 4):
        raise ValueError(f"the codebook format stores 2- or 4-bit codes, got n_bits={n_bits}")
    Layer = _layer_class()

    class _CompressedDynamicCache(DynamicCache):
        def __init__(self):
            super().__init__()
            self.n_bits = n_bits
            self.group_size = group_size
            self.head_dim = head_dim
            self.fused = fused
            self.layer_class_to_replicate = lambda: Layer(len(self.layers), n_bits, page_tokens, fused)

        def get_compressed_memory_bytes(self) -> int:
            return sum(layer.compressed_bytes() for layer in self.layers)

        def get_standard_memory_bytes(self) -> int:
            """Bytes the same positions would take as fp16 K + V."""
            total = 0
            for layer in self.layers:
                if layer.kc is not None:
                    total += 2 * layer.kc.batch * layer.kc.num_heads * layer.kc.seq_len * layer.kc.head_dim * 2
            return total

    _CompressedDynamicCache.__name__ = "CompressedDynamicCache"
    return _CompressedDynamicCache()


def patch_model(model, n_bits: int = 4, group_size: int = 32, fused: bool = True):
    """Record the compression settings on the model (hf_integration.py:93-118)
    and, with fused, switch its attention to polarquant_attention;
    create_compressed_cache(model) then builds the cache to pass as
    past_key_values."""
    cfg = model.config
    head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
    if fused:
        model.set_attn_implementation(register_attention())
    model._polarquant_config = {"n_bits": n_bits, "group_size": group_size, "head_dim": head_dim,
                                "num_layers": cfg.num_hidden_layers, "fused": fused}
    return model


def create_compressed_cache(model):
    c = model._polarquant_config
    fused = c["fused"] and getattr(model.config, "_attn_implementation", None) == ATTENTION_NAME
    return CompressedDynamicCache(n_bits=c["n_bits"], group_size=c["group_size"], head_dim=c["head_dim"],
                                  num_layers=c["num_layers"], fused=fused)
