"""GGML_TYPE_PQ4: the block format as a ggml type, and its HIP backend ops.

The reference's llama.cpp integration stores the cache as Q4_0 and never
calls its PolarQuant kernels from the graph (integration/polarquant-kv.patch:
1130-1137, 1303-1362, 1385-1404). This module is the ggml side done on
libpqkv_hip.so: the type's CPU traits (quantize / dequantize rows) and the two
backend ops a cache in it needs, cpy (f32 / f16 rows -> PQ4 rows) and
flash_attn_ext (attention of f32 queries over PQ4 keys and values with ggml's
additive mask). Tensors are passed as torch tensors whose dimensions are
ggml's in reverse order (torch [ne3, ne2, ne1, ne0]); any strides are kept
and handed to the library as ggml byte strides.

A PQ4 head of head_dim elements is rotated by the state's R (Gram-Schmidt
over rand() after srand(42), patch:549-579), stored as an fp16 radius (the
128-slot tree, csrc/flash_turboquant.cu:141-148) in each of its 18-byte
blocks and one 4-bit code per coordinate (the table of patch:978-983); its
value is (r16 c[code]) R.
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib

QK_PQ4 = 32          # elements per block (ggml blck_size)
TYPE_SIZE = 18       # bytes per block (ggml type_size)


def row_size(ne0: int) -> int:
    """Bytes of a PQ4 row of ne0 elements."""
    return ne0 // QK_PQ4 * TYPE_SIZE


def rotation(head_dim: int = 128) -> np.ndarray:
    """The type's rotation [head_dim, head_dim] float32 (what
    polarquant_init_c uploads)."""
    R = np.empty((head_dim, head_dim), np.float32)
    _lib.check(_lib.lib().pqkv_ggml_pq4_rotation(R.ctypes.data, head_dim))
    return R


def quantize_rows(x, head_dim: int = 128, R=None, codebook=None) -> np.ndarray:
    """CPU type trait: x float32 [..., k] (k whole heads) -> PQ4 rows uint8
    [..., row_size(k)]. R / codebook default to the type's own."""
    x = np.ascontiguousarray(x, np.float32)
    k = x.shape[-1]
    out = np.empty(x.shape[:-1] + (row_size(k),), np.uint8)
    if R is None and codebook is None and head_dim == 128:
        _lib.lib().pqkv_ggml_quantize_row_pq4_ref(x.ctypes.data, out.ctypes.data, x.size)
        return out
    Rm = np.ascontiguousarray(rotation(head_dim) if R is None else R, np.float32)
    cb = np.ascontiguousarray(default_codebook() if codebook is None else codebook, np.float32)
    _lib.check(_lib.lib().pqkv_pq4_quantize_rows_host(x.ctypes.data, out.ctypes.data, x.size, head_dim,
                                                      Rm.ctypes.data, cb.ctypes.data))
    return out


def dequantize_rows(y, k: int, head_dim: int = 128, R=None, codebook=None) -> np.ndarray:
    """CPU type trait: PQ4 rows uint8 [..., row_size(k)] -> float32 [..., k]."""
    y = np.ascontiguousarray(y, np.uint8)
    lead = y.shape[:-1]
    n = int(np.prod(lead)) * k if lead else k
    out = np.empty(lead + (k,), np.float32)
    if R is None and codebook is None and head_dim == 128:
        _lib.lib().pqkv_ggml_dequantize_row_pq4(y.ctypes.data, out.ctypes.data, n)
        return out
    Rm = np.ascontiguousarray(rotation(head_dim) if R is None else R, np.float32)
    cb = np.ascontiguousarray(default_codebook() if codebook is None else codebook, np.float32)
    _lib.check(_lib.lib().pqkv_pq4_dequantize_rows_host(y.ctypes.data, out.ctypes.data, n, head_dim,
                                                        Rm.ctypes.data, cb.ctypes.data))
    return out


def default_codebook() -> np.ndarray:
    """The type's 4-bit table: the one polarquant_init_c uploads and the
    default traits use (patch:978-983), a fixed input of the format."""
    return np.array([-0.1547, -0.1175, -0.0928, -0.0722, -0.0537, -0.0363, -0.0193, -0.0024,
                     0.0145, 0.0318, 0.0498, 0.0692, 0.0907, 0.1157, 0.1467, 0.1947], np.float32)


class _StateFields(ctypes.Structure):
    _fields_ = [("enabled", ctypes.c_int), ("n_bits", ctypes.c_int), ("n_levels", ctypes.c_int),
                ("head_dim", ctypes.c_int), ("n_kv_heads", ctypes.c_int), ("n_q_heads", ctypes.c_int),
                ("n_layers", ctypes.c_int), ("n_kv_max", ctypes.c_int), ("codebook", ctypes.c_void_p),
                ("rotation", ctypes.c_void_p), ("layers", ctypes.c_void_p)]


class State:
    """A 4-bit polarquant_state (polarquant_init_c) holding the type's
    rotation and codebook on the current device. Use as a context manager or
    call close()."""

    def __init__(self, head_dim: int = 128, n_kv_heads: int = 1, n_q_heads: int = 1):
        self.ptr = _lib.lib().polarquant_init_c(head_dim, n_kv_heads, n_q_heads, 1, 1, 4)
        if not self.ptr:
            raise RuntimeError("polarquant_init_c failed")
        self.head_dim = head_dim

    @property
    def fields(self) -> _StateFields:
        return _StateFields.from_address(self.ptr)

    def close(self) -> None:
        if self.ptr:
            _lib.lib().polarquant_free_c(self.ptr)
            self.ptr = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def _ne_nb(t, ne0=None, elt=None):
    """ggml ne / nb of a torch tensor of up to 4 dims (torch order reversed);
    for uint8 PQ4 rows ne0 is given and nb[0] is the block size."""
    shape = list(t.shape)[::-1] + [1] * (4 - t.dim())
    strides = [s * t.element_size() for s in list(t.stride())[::-1]] + [0] * (4 - t.dim())
    for i in range(t.dim(), 4):
        strides[i] = strides[i - 1] * shape[i - 1] if i > 0 else t.element_size()
    if ne0 is not None:
        shape[0] = ne0
        strides[0] = TYPE_SIZE if elt is None else elt
    return (_lib.c_int64_4)(*shape), (_lib.c_size_4)(*strides)


def cpy(state: State, src, dst) -> None:
    """src f32 / f16 [ne3, ne2, ne1, ne0] (any strides, contiguous rows) ->
    dst uint8 [ne3, ne2, ne1, row_size(ne0)] PQ4 rows (any row strides), on
    src's current stream."""
    _lib.require_device(src, dst)
    ne, nb = _ne_nb(src)
    if list(dst.shape[:-1]) != list(src.shape[:-1]) or dst.shape[-1] != row_size(src.shape[-1]):
        raise ValueError(f"dst {tuple(dst.shape)} does not hold PQ4 rows of src {tuple(src.shape)}")
    dne, dnb = _ne_nb(dst, ne0=src.shape[-1])
    _lib.check(_lib.lib().pqkv_ggml_cpy_pq4(state.ptr, src.data_ptr(), _lib.dtype_code(src.dtype), ne, nb,
                                            dst.data_ptr(), dnb, _lib.stream_of(src)))


def flash_attn_ext(state: State, q, k, v, mask=None, scale: float = 1.0, max_bias: float = 0.0,
                   logit_softcap: float = 0.0):
    """ggml_flash_attn_ext over PQ4 keys and values.

    q    f32   [n_seq, Hq, n_q, d]              (any strides, contiguous rows)
    k, v uint8 [n_seq_kv, Hkv, n_kv, row_size(d)] PQ4 heads (any strides;
               n_seq_kv 1 or n_seq)
    mask f16   [n_seq_m, 1, >= n_q, >= n_kv] additive, or None (n_seq_m 1 or n_seq)
    returns f32 [n_seq, n_q, Hq, d] (ggml's [d, Hq, n_q, n_seq])."""
    import torch
    _lib.require_device(q, k, v, mask)
    d = q.shape[-1]
    qne, qnb = _ne_nb(q)
    kne, knb = _ne_nb(k, ne0=d)
    vne, vnb = _ne_nb(v, ne0=d)
    if mask is not None:
        mne, mnb = _ne_nb(mask)
        mp = mask.data_ptr()
    else:
        mne, mnb, mp = None, None, None
    ns, Hq, n_q = q.shape[0], q.shape[1], q.shape[2]
    out = torch.empty((ns, n_q, Hq, d), dtype=torch.float32, device=q.device)
    L = _lib.lib()
    ws_bytes = L.pqkv_ggml_flash_attn_ext_pq4_workspace_bytes(state.ptr, qne, kne)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=q.device)
    _lib.check(L.pqkv_ggml_flash_attn_ext_pq4(state.ptr, q.data_ptr(), qne, qnb, k.data_ptr(), kne, knb,
                                              v.data_ptr(), vne, vnb, mp, mne, mnb, float(scale), float(max_bias),
                                              float(logit_softcap), out.data_ptr(), ws.data_ptr(), ws_bytes,
                                              _lib.stream_of(q)))
    return out


__all__ = ["QK_PQ4", "TYPE_SIZE", "row_size", "rotation", "quantize_rows", "dequantize_rows", "default_codebook",
           "State", "cpy", "flash_attn_ext"]
