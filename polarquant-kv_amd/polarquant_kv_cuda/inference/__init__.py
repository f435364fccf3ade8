"""Inference layer on the group format (src/polarquant_kv_cuda/inference)."""
