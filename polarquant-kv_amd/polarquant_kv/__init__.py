"""polarquant_kv - MI355X (gfx950) implementation of PolarQuant-KV's hot path.

Host-side mirror of the reference's Python interface (hilllief/polarquant-kv:
python/polarquant_kv and src/polarquant_kv_cuda) for the codebook
("TurboQuant") KV-cache path:

  rotation   generate_rotation_matrix, rotate, inverse_rotate
  lloyd_max  build_lloyd_max_codebook, quantize_with_codebook, ...
  qjl        generate_jl_matrix, bit_pack, bit_unpack
  quantizer  compress_pq, compress_gpu, decompress_gpu, ...    (HIP)
  attention  compressed_attention_gpu, compressed_attention, ... (HIP)
  turboquant turboquant_compress, turboquant_full_attention      (HIP, raw pointers)
  inference  PolarQuantConfig, KVCacheManager, CompressedMultiHeadAttention
  hf_integration CompressedDynamicCache, patch_model
  policies   compute_token_bitwidths, compute_layer_bitwidths, TokenMixedCache,
             differential_encode, ...                            (HIP for the cache)

GPU work goes through libpqkv_hip.so (include/pqkv.h) via ctypes.
"""

from . import lloyd_max, qjl, rotation, types  # noqa: F401
from .types import PQCache, block_bytes, vector_bytes  # noqa: F401

__all__ = ["lloyd_max", "qjl", "rotation", "types", "PQCache", "block_bytes", "vector_bytes"]


def __getattr__(name):
    # GPU modules load libpqkv_hip.so lazily so the host-side API imports
    # on machines without a GPU.
    if name in ("attention", "quantizer", "turboquant", "inference", "hf_integration", "policies"):
        import importlib
        return importlib.import_module(f".{name}", __name__)
    raise AttributeError(name)
