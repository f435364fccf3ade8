"""QJL sign sketch on the GPU (src/polarquant_kv_cuda/qjl_kernel.py:6-135):
compute_signatures_gpu runs pqkv_qjl_sketch (signs of P e summed in fp64,
packed LSB first, and |e|); the correction and the bit packing helpers are
those of polarquant_kv.qjl."""

from __future__ import annotations

from polarquant_kv.qjl import bit_pack, bit_unpack, compute_correction_gpu, compute_signatures_gpu  # noqa: F401


def _batch_bit_pack(signs):
    """[..., m] bool -> [..., ceil(m/8)] uint8 (qjl_kernel.py:112-124)."""
    return bit_pack(signs)


def _batch_bit_unpack(packed, jl_dim: int):
    """[..., ceil(m/8)] uint8 -> [..., m] bool (qjl_kernel.py:127-135)."""
    return bit_unpack(packed, jl_dim)
