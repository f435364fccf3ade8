"""The polarquant_kv_cuda import surface: every name the reference's own files
import from src/polarquant_kv_cuda (scripts/benchmark_turboquant.py:9-12,
scripts/benchmark_innovations.py:3-9, scripts/e2e_qwen_compressed.py:10-12,
tests/cuda/*.py) resolves here, as do the module names of its pybind
extensions polarquant_turboquant and polarquant_full. Out of scope and absent:
the cupy / PTX modules (fused_attention*, fused_cuda_kernels,
flash_attention_native, cuda_native) and the Windows-only polarquant_native."""

import importlib

import pytest

SURFACE = {
    "polarquant_kv_cuda.rotation": ["generate_rotation_matrix", "rotate", "inverse_rotate"],
    "polarquant_kv_cuda.lloyd_max": ["build_lloyd_max_codebook", "quantize_with_codebook",
                                     "dequantize_with_codebook", "get_codebook_torch"],
    "polarquant_kv_cuda.types": ["CompressedKVCacheGPU"],
    "polarquant_kv_cuda.compress_kernel": ["compress_gpu", "_bit_pack_quantized", "_bit_unpack_quantized",
                                           "_packed_dim", "_validate_params"],
    "polarquant_kv_cuda.decompress_kernel": ["decompress_gpu"],
    "polarquant_kv_cuda.attention_kernel": ["compressed_attention_gpu"],
    "polarquant_kv_cuda.qjl_kernel": ["compute_signatures_gpu", "compute_correction_gpu", "bit_pack", "bit_unpack",
                                      "_batch_bit_pack", "_batch_bit_unpack"],
    "polarquant_kv_cuda.compressor": ["compress", "decompress", "compressed_attention", "get_memory_bytes"],
    "polarquant_kv_cuda.utils": ["cosine_similarity_gpu"],
    "polarquant_kv_cuda.inference.config": ["PolarQuantConfig"],
    "polarquant_kv_cuda.inference.kv_cache": ["KVCacheManager"],
    "polarquant_kv_cuda.inference.attention": ["CompressedMultiHeadAttention"],
    "polarquant_kv_cuda.inference.transformer": ["SimpleTransformer", "SimpleTransformerLayer"],
    "polarquant_kv_cuda.hf_integration": ["CompressedDynamicCache", "patch_model", "create_compressed_cache"],
    "polarquant_kv_cuda.token_importance": ["compute_token_bitwidths", "estimate_mixed_compression_ratio",
                                            "mixed_precision_compress"],
    "polarquant_kv_cuda.adaptive_bitwidth": ["compute_layer_bitwidths", "estimate_adaptive_compression_ratio"],
    "polarquant_kv_cuda.cross_layer": ["measure_cross_layer_similarity", "differential_encode",
                                       "differential_decode", "estimate_differential_gain"],
    "polarquant_turboquant": ["turboquant_compress", "turboquant_full_attention"],
    "polarquant_full": ["full_compressed_attention"],
}


@pytest.mark.parametrize("module", sorted(SURFACE))
def test_reference_names_resolve(module):
    mod = importlib.import_module(module)
    missing = [n for n in SURFACE[module] if not hasattr(mod, n)]
    assert not missing, missing


def test_dataclass_fields_are_the_reference_fields():
    from dataclasses import fields

    from polarquant_kv_cuda.types import CompressedKVCacheGPU
    assert [f.name for f in fields(CompressedKVCacheGPU)] == [
        "radius", "quantized_direction", "group_mins", "group_scales", "qjl_signs", "residual_norms", "n_bits",
        "group_size", "original_dim", "seq_len", "max_seq_len"]


def test_bit_pack_helpers_match_the_oracle():
    import numpy as np
    import torch

    from oracle import oracle as O
    from polarquant_kv_cuda.compress_kernel import _bit_pack_quantized, _bit_unpack_quantized, _packed_dim
    rng = np.random.default_rng(0)
    for bits in (2, 3, 4, 8):
        c = rng.integers(0, 1 << bits, size=(3, 64)).astype(np.uint8)
        p = _bit_pack_quantized(torch.from_numpy(c), bits)
        assert np.array_equal(p.numpy(), O.gpu_group_pack(c, bits))
        assert p.shape[-1] == _packed_dim(64, bits)
        assert np.array_equal(_bit_unpack_quantized(p, bits, 64).numpy(), c)
