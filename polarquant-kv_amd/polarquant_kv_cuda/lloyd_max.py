"""Lloyd-Max codebooks (src/polarquant_kv_cuda/lloyd_max.py:12-104)."""

from polarquant_kv.lloyd_max import (build_lloyd_max_codebook, dequantize_with_codebook,  # noqa: F401
                                     get_codebook_torch, quantize_with_codebook)
