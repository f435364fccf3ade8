"""ctypes binding of libpqkv_hip.so (the C ABI declared in include/pqkv.h).

The GPU entry points of this package call only through this module. If the
library is missing the import of any GPU entry point raises: there is no CPU
fallback for the hot path.
"""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# PQKV_LIBRARY selects another build of the library (same ABI), e.g. one
# compiled with different kernel options
LIB_PATH = os.environ.get("PQKV_LIBRARY") or os.path.join(_HERE, "_lib", "libpqkv_hip.so")

OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_WORKSPACE, ERR_HIP = 0, -1, -2, -3, -4
F32, F16, BF16 = 0, 1, 2

c_void_p, c_int, c_int64, c_float, c_size_t = (ctypes.c_void_p, ctypes.c_int, ctypes.c_int64,
                                               ctypes.c_float, ctypes.c_size_t)
c_int_p, c_float_p = ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_float)
c_int64_4, c_size_4 = ctypes.c_int64 * 4, ctypes.c_size_t * 4      # ggml ne / nb arrays
c_int64_p, c_size_p = ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_size_t)

# name -> (restype, argtypes); the full exported surface of include/pqkv.h
SIGNATURES = {
    "pqkv_version": (c_int, []),
    "pqkv_status_string": (ctypes.c_char_p, [c_int]),
    "pqkv_last_error": (ctypes.c_char_p, []),
    "pqkv_block_bytes": (c_int, [c_int]),
    "pqkv_vector_bytes": (c_int64, [c_int, c_int]),
    "pqkv_lloyd_max_codebook": (c_int, [c_int, c_int, c_int, c_int, c_void_p, c_void_p]),
    "pqkv_rotate": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_int, c_int64, c_int, c_int, c_void_p]),
    "pqkv_quantize_rotated": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_int64, c_int, c_void_p]),
    "pqkv_encode": (c_int, [c_void_p, c_int, c_int64, c_void_p, c_void_p, c_int, c_void_p, c_int64,
                            c_int64, c_int64, c_int, c_void_p, c_int, c_void_p, c_int64, c_void_p]),
    "pqkv_encode_mfma": (c_int, [c_void_p, c_int, c_int64, c_void_p, c_void_p, c_int, c_void_p, c_int64,
                                 c_int64, c_int64, c_int, c_void_p, c_void_p, c_void_p]),
    "pqkv_decode_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "pqkv_decode_attn": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                 c_int, c_int, c_int_p, c_int_p, c_void_p, c_void_p, c_int,
                                 c_int, c_int, c_int, c_int, c_int, c_int, c_float,
                                 c_void_p, c_int, c_void_p, c_size_t, c_void_p]),
    "pqkv_decode_attn_noalloc": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                         c_int, c_int, c_int_p, c_int_p, c_void_p, c_void_p, c_int,
                                         c_int, c_int, c_int, c_int, c_int, c_int, c_float,
                                         c_void_p, c_int, c_void_p]),
    "pqkv_decode_segments_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int_p, c_int]),
    "pqkv_decode_attn_segments": (c_int, [c_void_p, c_int, c_void_p, c_int,
                                          ctypes.POINTER(c_void_p), ctypes.POINTER(c_void_p),
                                          ctypes.POINTER(c_void_p), ctypes.POINTER(c_void_p),
                                          c_int_p, c_int_p, c_int_p, c_int_p,
                                          c_int, c_int, c_int, c_int, c_float,
                                          c_void_p, c_int, c_void_p, c_size_t, c_void_p]),
    "pqkv_encode_paged": (c_int, [c_void_p, c_int, c_int64, c_void_p, c_void_p, c_int, c_void_p, c_int, c_int,
                                  c_int64, c_int64, c_int64, c_int, c_void_p, c_int, c_void_p, c_void_p]),
    "pqkv_decode_attn_paged": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p,
                                       c_void_p, c_int, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                       c_int, c_float, c_void_p, c_int, c_void_p, c_size_t, c_void_p]),
    "pqkv_prefill_attn_paged": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p,
                                        c_void_p, c_int, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
                                        c_int, c_int, c_int, c_float, c_int, c_void_p, c_int, c_void_p, c_size_t,
                                        c_void_p]),
    "pqkv_group_compress": (c_int, [c_void_p, c_int, c_void_p, c_int64, c_int, c_int, c_int,
                                    c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "pqkv_group_decompress": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int,
                                      c_void_p, c_void_p]),
    "pqkv_group_gpu_compress": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_int64, c_int, c_int, c_int,
                                        c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p]),
    "pqkv_group_gpu_decompress": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_int64, c_int,
                                          c_int, c_int, c_void_p, c_int, c_void_p]),
    "pqkv_qjl_sketch": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_int64, c_int, c_int, c_void_p, c_void_p,
                                c_int, c_void_p]),
    "pqkv_group_attn_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int, c_int, c_int]),
    "pqkv_group_attn": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_void_p, c_int,
                                c_void_p, c_size_t, c_void_p]),
    "pqkv_soa_attn_generic_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int]),
    "pqkv_soa_attn_generic": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                      c_int, c_int, c_int, c_float, c_void_p, c_void_p, c_size_t, c_void_p]),
    "pqkv_prefill_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int, c_int]),
    "pqkv_prefill_attn": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                  c_int, c_int, c_int_p, c_int_p, c_void_p, c_void_p, c_int,
                                  c_int, c_int, c_int, c_int, c_int, c_int, c_int,
                                  c_int, c_float, c_int, c_void_p, c_int, c_void_p, c_size_t, c_void_p]),
    "pqkv_dequantize": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_int, c_int64, c_int, c_void_p]),
    "pqkv_soa_to_blocks": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int, c_void_p]),
    "pqkv_blocks_to_soa": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int, c_void_p]),
    "pqkv_profile_enable": (c_int, [c_int]),
    "pqkv_profile_repeat": (c_int, [c_int]),
    "pqkv_profile_stream_read": (c_int, [c_void_p, c_size_t, c_void_p, c_int, c_void_p]),
    "pqkv_profile_collect": (c_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_double),
                                     ctypes.POINTER(ctypes.c_int64)]),
    "polarquant_init_c": (c_void_p, [c_int, c_int, c_int, c_int, c_int, c_int]),
    "polarquant_free_c": (None, [c_void_p]),
    "polarquant_compress_cuda_c": (None, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                          c_int, c_void_p]),
    "polarquant_rotate_query_cuda_c": (None, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "polarquant_fused_attention_cuda_c": (None, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                                 c_void_p, c_int, c_int, c_int, c_int, c_int, c_float,
                                                 c_void_p]),
    "polarquant_inverse_rotate_cuda_c": (None, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_void_p]),
    "turboquant_compress": (None, [c_int64] * 5 + [c_int] * 3),
    "turboquant_full_attention": (None, [c_int64] * 12 + [c_int] * 5 + [c_float]),
    "full_compressed_attention": (None, [c_int64] * 14 + [c_int] * 6 + [c_float]),
    "pqkv_pq4_quantize_rows_host": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_void_p, c_void_p]),
    "pqkv_pq4_dequantize_rows_host": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_void_p, c_void_p]),
    "pqkv_ggml_pq4_rotation": (c_int, [c_void_p, c_int]),
    "pqkv_ggml_quantize_row_pq4_ref": (None, [c_void_p, c_void_p, c_int64]),
    "pqkv_ggml_dequantize_row_pq4": (None, [c_void_p, c_void_p, c_int64]),
    "pqkv_ggml_cpy_pq4": (c_int, [c_void_p, c_void_p, c_int, c_int64_p, c_size_p, c_void_p, c_size_p, c_void_p]),
    "pqkv_ggml_flash_attn_ext_pq4_workspace_bytes": (c_size_t, [c_void_p, c_int64_p, c_int64_p]),
    "pqkv_ggml_flash_attn_ext_pq4": (c_int, [c_void_p, c_void_p, c_int64_p, c_size_p, c_void_p, c_int64_p, c_size_p,
                                             c_void_p, c_int64_p, c_size_p, c_void_p, c_int64_p, c_size_p,
                                             c_float, c_float, c_float, c_void_p, c_void_p, c_size_t,
                                             c_void_p]),
}

_lib = None


class PQKVError(RuntimeError):
    """A C-ABI call returned a negative status."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{message} (status {status})")
        self.status = status


def lib() -> ctypes.CDLL:
    """Load libpqkv_hip.so once; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with "
                              "`python polarquant-kv_amd/build_lib.py` (the HIP path has no CPU fallback)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status: int) -> None:
    if status != OK:
        raise PQKVError(status, lib().pqkv_last_error().decode())


def dtype_code(t) -> int:
    import torch
    if t == torch.float32:
        return F32
    if t == torch.float16:
        return F16
    raise TypeError(f"unsupported dtype {t} (float32 or float16)")


def stream_of(t) -> int:
    """The current torch stream of the tensor's device, as a hipStream_t."""
    import torch
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def require_device(*tensors) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("GPU entry points take device tensors (the hot path has no CPU fallback)")


def ptr_array(tensors):
    """Host array of the tensors' device pointers (for the segment arrays)."""
    return (c_void_p * len(tensors))(*[t.data_ptr() for t in tensors])


def int_array(values):
    if values is None:
        return None
    arr = (ctypes.c_int * len(values))(*[int(v) for v in values])
    return arr


def profile_enable(on: bool = True) -> None:
    check(lib().pqkv_profile_enable(int(on)))


def profile_repeat(n: int) -> None:
    check(lib().pqkv_profile_repeat(int(n)))


def profile_collect(name: str):
    """(total ms, launches) of the profiled kernels whose name contains `name`."""
    ms = ctypes.c_double(0.0)
    n = ctypes.c_int64(0)
    check(lib().pqkv_profile_collect(name.encode(), ctypes.byref(ms), ctypes.byref(n)))
    return ms.value, n.value
