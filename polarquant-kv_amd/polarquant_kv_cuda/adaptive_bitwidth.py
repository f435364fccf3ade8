"""Per-layer bit widths (src/polarquant_kv_cuda/adaptive_bitwidth.py:15-83)."""

from polarquant_kv.policies import compute_layer_bitwidths, estimate_adaptive_compression_ratio  # noqa: F401
