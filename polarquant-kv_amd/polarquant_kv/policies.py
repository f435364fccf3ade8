"""Mixed-precision policies and the per-token mixed cache they feed.

Mirrors the reference's policy modules with the same names and arguments:

  token_importance   compute_token_bitwidths, mixed_precision_compress,
                     estimate_mixed_compression_ratio
                     (src/polarquant_kv_cuda/token_importance.py:17-90)
  adaptive_bitwidth  compute_layer_bitwidths, estimate_adaptive_compression_ratio
                     (src/polarquant_kv_cuda/adaptive_bitwidth.py:15-83)
  cross_layer        measure_cross_layer_similarity, differential_encode,
                     differential_decode, estimate_differential_gain
                     (src/polarquant_kv_cuda/cross_layer.py:17-102)

The reference's mixed_precision_compress only counts the tokens of each
width; here it also builds the cache: TokenMixedCache keeps the high-width
tokens (sinks and the recent window) and the low-width ones as two PQ caches
and attends on both with one softmax (pqkv_decode_attn_segments: both
segments' split partials go through one merge). Token order does not matter
to decode attention, so each segment stores its tokens contiguously.
"""

from __future__ import annotations

import torch

from . import _lib, quantizer
from .types import vector_bytes


# ---------------------------------------------------------------- per token

def compute_token_bitwidths(seq_len: int, sink_size: int = 4, window_size: int = 64, high_bits: int = 4,
                            low_bits: int = 2) -> torch.Tensor:
    """[seq_len] int32 widths: the first sink_size tokens and the last
    window_size tokens high_bits, the rest low_bits; a sequence no longer
    than sink_size + window_size is all high_bits
    (token_importance.py:17-40). As there, window_size = 0 marks every token
    high (the reference's slice bits[-0:] is the whole sequence)."""
    bits = torch.full((seq_len,), low_bits, dtype=torch.int32)
    bits[:min(sink_size, seq_len)] = high_bits
    if seq_len > sink_size + window_size:
        bits[seq_len - window_size if window_size > 0 else 0:] = high_bits
    elif seq_len > sink_size:
        bits[sink_size:] = high_bits
    return bits


def estimate_mixed_compression_ratio(seq_len: int, sink_size: int = 4, window_size: int = 64) -> float:
    """16 / mean width of compute_token_bitwidths (token_importance.py:82-89)."""
    bits = compute_token_bitwidths(seq_len, sink_size, window_size)
    return 16.0 / bits.float().mean().item()


class TokenMixedCache:
    """K and V of [B, H, S, d] split by per-token width into a high-width and
    a low-width PQ cache (device), attended on together."""

    def __init__(self, keys: list, values: list, rotation_matrix: torch.Tensor, positions: list, bits: list):
        self.keys = keys                  # PQCache per segment (high, low); None when empty
        self.values = values
        self.R = rotation_matrix
        self.positions = positions        # token indices of each segment (CPU int64)
        self.bits = bits                  # width of each segment

    @classmethod
    def from_kv(cls, keys: torch.Tensor, values: torch.Tensor, rotation_matrix: torch.Tensor,
                token_bits: torch.Tensor, codebooks: dict | None = None) -> "TokenMixedCache":
        """keys / values [B, H, S, d] (device, fp16/fp32); token_bits [S]
        with values 4 and 2. codebooks: optional {bits: table} overriding the
        Lloyd-Max tables of each width."""
        _lib.require_device(keys, values, rotation_matrix)
        if keys.shape != values.shape or keys.dim() != 4:
            raise ValueError("keys and values must both be [B, H, S, d]")
        S = keys.shape[2]
        tb = torch.as_tensor(token_bits).to("cpu", torch.int64)
        if tb.shape != (S,):
            raise ValueError(f"token_bits must have one width per token ({S}), got {tuple(tb.shape)}")
        widths = sorted({int(b) for b in tb.tolist()}, reverse=True)
        if any(b not in (2, 4) for b in widths):
            raise ValueError(f"token widths must be 2 or 4, got {widths}")
        B, H, _, d = keys.shape
        kcs, vcs, pos = [], [], []
        for b in widths:
            idx = torch.nonzero(tb == b).flatten()
            dev_idx = idx.to(keys.device)
            table = None
            if codebooks and b in codebooks:
                table = torch.zeros(16, dtype=torch.float32, device=keys.device)
                cb = torch.as_tensor(codebooks[b], dtype=torch.float32, device=keys.device).flatten()
                table[:cb.numel()] = cb
            kc = quantizer.allocate_cache(B, H, len(idx), d, b, keys.device, codebooks=table)
            vc = quantizer.allocate_cache(B, H, len(idx), d, b, keys.device, codebooks=table)
            quantizer.compress_pq(keys.index_select(2, dev_idx).contiguous(), rotation_matrix, cache=kc, start=0)
            quantizer.compress_pq(values.index_select(2, dev_idx).contiguous(), rotation_matrix, cache=vc, start=0)
            kcs.append(kc)
            vcs.append(vc)
            pos.append(idx)
        return cls(kcs, vcs, rotation_matrix, pos, widths)

    @property
    def seq_len(self) -> int:
        return sum(c.seq_len for c in self.keys)

    @property
    def memory_bytes(self) -> int:
        return sum(c.memory_bytes() for c in self.keys) + sum(c.memory_bytes() for c in self.values)

    @property
    def avg_bits(self) -> float:
        n = self.seq_len
        return sum(b * len(p) for b, p in zip(self.bits, self.positions)) / n if n else 0.0

    def attend(self, query: torch.Tensor, scale: float | None = None, out_dtype=torch.float16) -> torch.Tensor:
        """query [B, Hq, d] (one token per sequence) -> [B, Hq, d]: decode
        attention over every cached token of both widths."""
        from .attention import decode_attention_segments
        return decode_attention_segments(query, list(zip(self.keys, self.values)), self.R, scale=scale,
                                         out_dtype=out_dtype)


def mixed_precision_compress(kv: torch.Tensor, rotation_matrix: torch.Tensor, codebook_4bit: torch.Tensor,
                             codebook_2bit: torch.Tensor, token_bits: torch.Tensor, values: torch.Tensor | None = None
                             ) -> dict:
    """Per-token mixed-precision compression (token_importance.py:43-79):
    the reference's statistics (n_high, n_low, avg_bits, compression_ratio,
    high_mask, low_mask) and, under "cache", the TokenMixedCache of kv (as
    keys and, unless `values` is given, as values) with the given codebooks."""
    tb = torch.as_tensor(token_bits).to("cpu")
    B, H, S, D = kv.shape
    high_mask = tb == 4
    low_mask = tb == 2
    n_high = int(high_mask.sum().item())
    n_low = int(low_mask.sum().item())
    avg_bits = (n_high * 4 + n_low * 2) / S
    cache = TokenMixedCache.from_kv(kv, kv if values is None else values, rotation_matrix, tb,
                                    codebooks={4: codebook_4bit, 2: codebook_2bit})
    return {"n_high": n_high, "n_low": n_low, "avg_bits": avg_bits, "compression_ratio": 16.0 / avg_bits,
            "high_mask": high_mask, "low_mask": low_mask, "cache": cache}


# ---------------------------------------------------------------- per layer

def compute_layer_bitwidths(num_layers: int, target_avg_bits: float = 3.0, min_bits: int = 2,
                            max_bits: int = 4) -> list:
    """U-shaped per-layer widths (adaptive_bitwidth.py:15-68): width
    min + |i - mid| / mid * (max - min) rounded half to even, then, if the
    mean exceeds target_avg_bits, one bit off each layer in order of
    increasing distance from the middle until it does not."""
    if num_layers <= 2:
        return [max_bits] * num_layers
    mid = (num_layers - 1) / 2.0
    weights = [abs(i - mid) / mid for i in range(num_layers)]
    widths = [max(min_bits, min(max_bits, round(min_bits + w * (max_bits - min_bits)))) for w in weights]
    if sum(widths) / num_layers > target_avg_bits:
        for i in sorted(range(num_layers), key=lambda x: weights[x]):
            if widths[i] > min_bits:
                widths[i] -= 1
                if sum(widths) / num_layers <= target_avg_bits:
                    break
    return widths


def estimate_adaptive_compression_ratio(bitwidths: list, head_dim: int = 128) -> float:
    """16 / mean over layers of (bits + 128 / head_dim), the reference's
    estimate with an fp32 radius per 32 values (adaptive_bitwidth.py:71-83)."""
    total = sum(b + 4.0 / head_dim * 32 for b in bitwidths)
    return 16.0 / (total / len(bitwidths))


# ---------------------------------------------------------------- cross layer

def measure_cross_layer_similarity(kv_layers: list) -> list:
    """Per adjacent layer pair: mean cosine similarity of the vectors and the
    mean difference norm over the mean norm (cross_layer.py:17-54)."""
    out = []
    for i in range(1, len(kv_layers)):
        prev = kv_layers[i - 1].float()
        curr = kv_layers[i].float()
        d = prev.shape[-1]
        cos = torch.nn.functional.cosine_similarity(prev.reshape(-1, d), curr.reshape(-1, d), dim=1).mean().item()
        diff_norm = (curr - prev).norm(dim=-1).mean().item()
        orig_norm = curr.norm(dim=-1).mean().item()
        out.append({"layer": i, "cosine_similarity": cos, "diff_norm_ratio": diff_norm / (orig_norm + 1e-10)})
    return out


def differential_encode(kv_layers: list) -> list:
    """Layer 0 as is, layer i as layer i - layer (i - 1) (cross_layer.py:57-69)."""
    return [kv_layers[0]] + [kv_layers[i] - kv_layers[i - 1] for i in range(1, len(kv_layers))]


def differential_decode(encoded_layers: list) -> list:
    """Running sum of differential_encode's output (cross_layer.py:72-80)."""
    out = [encoded_layers[0]]
    for i in range(1, len(encoded_layers)):
        out.append(out[i - 1] + encoded_layers[i])
    return out


def estimate_differential_gain(num_layers: int, avg_diff_norm_ratio: float = 0.4) -> float:
    """The reference's heuristic gain (cross_layer.py:83-102):
    1 / (1 - 0.3 (1 - ratio)(L - 1) / L)."""
    savings = (1.0 - avg_diff_norm_ratio) * (num_layers - 1) / num_layers
    return 1.0 / (1.0 - savings * 0.3)


def layer_cache_bytes(num_tokens: int, head_dim: int, bitwidths: list) -> int:
    """Bytes of K + V per layer-width list for num_tokens vectors per layer
    in the block format (2 or 4 bits; fp16 radius per 32 coordinates)."""
    return sum(2 * num_tokens * vector_bytes(head_dim, b) for b in bitwidths)


__all__ = ["compute_token_bitwidths", "estimate_mixed_compression_ratio", "mixed_precision_compress",
           "TokenMixedCache", "compute_layer_bitwidths", "estimate_adaptive_compression_ratio",
           "measure_cross_layer_similarity", "differential_encode", "differential_decode",
           "estimate_differential_gain", "layer_cache_bytes"]
