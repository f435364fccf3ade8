"""Per-token mixed precision (src/polarquant_kv_cuda/token_importance.py:17-90)."""

from polarquant_kv.policies import (TokenMixedCache, compute_token_bitwidths,  # noqa: F401
                                    estimate_mixed_compression_ratio, mixed_precision_compress)
