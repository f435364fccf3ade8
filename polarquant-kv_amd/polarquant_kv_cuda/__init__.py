"""polarquant_kv_cuda - the reference's GPU-side Python package
(src/polarquant_kv_cuda of hilllief/polarquant-kv) on MI355X.

Module names follow the reference, so callers switch by import path alone.
What each module computes on (libpqkv_hip.so through polarquant_kv._lib):

  types              CompressedKVCacheGPU (the reference's fields)
  rotation           generate_rotation_matrix, rotate, inverse_rotate
  lloyd_max          build_lloyd_max_codebook, quantize_with_codebook,
                     dequantize_with_codebook, get_codebook_torch
  compress_kernel    compress_gpu: the group (min / scale) format, on the GPU
  decompress_kernel  decompress_gpu: fp16 reconstruction, on the GPU
  attention_kernel   compressed_attention_gpu: attention straight on the
                     group-format caches (fused kernel), or on PQCache
                     (codebook format) caches
  qjl_kernel         compute_signatures_gpu, compute_correction_gpu, bit packing
  compressor         compress, decompress, compressed_attention, get_memory_bytes
  utils              cosine_similarity_gpu
  inference          PolarQuantConfig, KVCacheManager, CompressedMultiHeadAttention,
                     SimpleTransformerLayer, SimpleTransformer (group format,
                     the reference's semantics; preallocated in-place appends)
  hf_integration     CompressedDynamicCache, patch_model, create_compressed_cache
                     (the codebook format of polarquant_kv.hf_integration)
  token_importance, adaptive_bitwidth, cross_layer
                     the mixed-precision policy functions (polarquant_kv.policies)
"""
