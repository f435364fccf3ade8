"""Hugging Face transformers integration (transformers 5 cache API).

Mirrors src/polarquant_kv_cuda/hf_integration.py of the reference
(CompressedDynamicCache, patch_model, create_compressed_cache) with one
difference in kind: the reference's cache keeps the model's fp16 states and
adds compressed copies that nothing reads (hf_integration.py:43-62), so the
model still attends on the original states. Here each layer keeps only the
compressed cache (block_pq4 / block_pq2, encoded in place on every update by
the HIP encoder, with the reference's per-layer rotation seeds 42 + layer)
and returns its reconstruction r16 * c[code] R (the HIP dequantise kernel),
so the model attends on the compressed representation and the resident cache
is the compressed one. Capacity grows in pages of tokens (page_tokens) as
the sequence grows.
"""

from __future__ import annotations

import torch

from . import quantizer
from .types import PQCache


def _cache_utils():
    try:
        from transformers.cache_utils import DynamicCache, DynamicLayer
    except ImportError as e:            # pragma: no cover - transformers is optional
        raise ImportError("the Hugging Face integration needs transformers >= 5") from e
    return DynamicCache, DynamicLayer


def _layer_class():
    _, DynamicLayer = _cache_utils()

    class CompressedLayer(DynamicLayer):
        """One layer of CompressedDynamicCache."""

        def __init__(self, layer_idx: int, n_bits: int, page_tokens: int):
            super().__init__()
            self.layer_idx = layer_idx
            self.n_bits = n_bits
            self.page_tokens = page_tokens
            self.kc: PQCache | None = None
            self.vc: PQCache | None = None
            self.R = None

        def lazy_initialization(self, key_states, value_states, *args, **kwargs):
            from .rotation import generate_rotation_matrix
            self.dtype, self.device = key_states.dtype, key_states.device
            self.R = generate_rotation_matrix(key_states.shape[-1], seed=42 + self.layer_idx, device=self.device)
            # the layer keeps no fp16 states
            self.keys = torch.empty(0, dtype=self.dtype, device=self.device)
            self.values = torch.empty(0, dtype=self.dtype, device=self.device)
            self.is_initialized = True

        def _ensure_capacity(self, B, H, need, d):
            cap = self.kc.max_seq_len if self.kc is not None else 0
            if need <= cap:
                return
            new_cap = max(need, 2 * cap, self.page_tokens)
            new_cap = (new_cap + self.page_tokens - 1) // self.page_tokens * self.page_tokens
            kc = quantizer.allocate_cache(B, H, new_cap, d, self.n_bits, self.device)
            vc = quantizer.allocate_cache(B, H, new_cap, d, self.n_bits, self.device)
            if self.kc is not None:
                S = self.kc.seq_len
                kc.blocks[:, :, :S] = self.kc.blocks[:, :, :S]
                vc.blocks[:, :, :S] = self.vc.blocks[:, :, :S]
                kc.seq_len = vc.seq_len = S
            self.kc, self.vc = kc, vc

        def update(self, key_states, value_states, *args, **kwargs):
            if not self.is_initialized:
                self.lazy_initialization(key_states, value_states)
            B, H, T, d = key_states.shape
            start = self.get_seq_length()
            self._ensure_capacity(B, H, start + T, d)
            quantizer.compress_pq(key_states.contiguous(), self.R, cache=self.kc, start=start)
            quantizer.compress_pq(value_states.contiguous(), self.R, cache=self.vc, start=start)
            keys = quantizer.dequantize(self.kc, self.R, self.dtype if self.dtype in (torch.float16, torch.float32)
                                        else torch.float32)
            values = quantizer.dequantize(self.vc, self.R, keys.dtype)
            return keys.to(self.dtype), values.to(self.dtype)

        def get_seq_length(self) -> int:
            return 0 if self.kc is None else self.kc.seq_len

        def get_mask_sizes(self, query_length: int, *args, **kwargs):
            return self.get_seq_length() + query_length, 0

        def crop(self, tokens_to_remove: int) -> None:
            """DynamicLayer.crop's rule (transformers 5): a negative value
            removes that many tokens, a positive one is the legacy absolute
            length to keep (nothing happens when it is not below the current
            length), and 0 does nothing."""
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

        def batch_repeat_interleave(self, repeats: int):
            raise NotImplementedError("beam expansion of a compressed cache")

        def batch_select_indices(self, indices):
            raise NotImplementedError("beam selection of a compressed cache")

        def reorder_cache(self, beam_idx):
            raise NotImplementedError("beam reordering of a compressed cache")

    return CompressedLayer


def CompressedDynamicCache(n_bits: int = 4, group_size: int = 32, head_dim: int | None = None,
                           num_layers: int | None = None, page_tokens: int = 256):
    """A transformers DynamicCache whose layers store only the PQ-encoded
    keys and values (hf_integration.py:21 of the reference keeps the same
    constructor arguments; head_dim and num_layers are taken from the states
    as they arrive, and group_size is checked like the reference's)."""
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
            self.layer_class_to_replicate = lambda: Layer(len(self.layers), n_bits, page_tokens)

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


def patch_model(model, n_bits: int = 4, group_size: int = 32):
    """Record the compression settings on the model
    (hf_integration.py:93-118); create_compressed_cache(model) then builds
    the cache to pass as past_key_values."""
    cfg = model.config
    head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // cfg.num_attention_heads
    model._polarquant_config = {"n_bits": n_bits, "group_size": group_size, "head_dim": head_dim,
                                "num_layers": cfg.num_hidden_layers}
    return model


def create_compressed_cache(model):
    c = model._polarquant_config
    return CompressedDynamicCache(n_bits=c["n_bits"], group_size=c["group_size"], head_dim=c["head_dim"],
                                  num_layers=c["num_layers"])
