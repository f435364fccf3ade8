"""Hugging Face cache (src/polarquant_kv_cuda/hf_integration.py:21-127): the
codebook-format cache of polarquant_kv.hf_integration, which attends through
the fused decode / prefill kernels."""

from polarquant_kv.hf_integration import CompressedDynamicCache, create_compressed_cache, patch_model  # noqa: F401
