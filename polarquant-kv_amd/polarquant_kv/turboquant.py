"""The reference's raw-pointer binding, polarquant_turboquant
(csrc/flash_turboquant.cu:227-230), on libpqkv_hip.so.

Callers pass device pointers as Python ints, exactly as
scripts/benchmark_turboquant.py:88-114 does with the reference module:

    turboquant_compress(input, R, cb, radius_out, packed_out, N, D, n_levels)
    turboquant_full_attention(q, R, pk, kr, pv, vr, k_cb, v_cb, out, q_rot,
                              score, attn_out, total_heads, total_kv, S, D,
                              n_levels, scale)

Both return None and run asynchronously on the null stream (the caller
synchronises), like the reference. Buffers are caller-owned; keep the tensors
alive until the work has run. The SoA layout is the reference's: packed
codes [N][D/2] (coordinate 2i in the low nibble) and fp32 radii [N].
turboquant_full_attention reads the rotated queries at q_rot and writes the
rotated output to attn_out; q, R and out are not read (flash_turboquant.cu:
188-209).
"""

from __future__ import annotations

from . import _lib


def turboquant_compress(input_ptr: int, R_ptr: int, cb_ptr: int, radius_ptr: int, packed_ptr: int, N: int,
                        D: int, n_levels: int) -> None:
    _lib.lib().turboquant_compress(int(input_ptr), int(R_ptr), int(cb_ptr), int(radius_ptr), int(packed_ptr),
                                   int(N), int(D), int(n_levels))


def turboquant_full_attention(q_ptr: int, R_ptr: int, pk_ptr: int, kr_ptr: int, pv_ptr: int, vr_ptr: int,
                              k_cb_ptr: int, v_cb_ptr: int, out_ptr: int, q_rot_ptr: int, score_ptr: int,
                              attn_out_ptr: int, total_heads: int, total_kv: int, S: int, D: int, n_levels: int,
                              scale: float) -> None:
    _lib.lib().turboquant_full_attention(int(q_ptr), int(R_ptr), int(pk_ptr), int(kr_ptr), int(pv_ptr),
                                         int(vr_ptr), int(k_cb_ptr), int(v_cb_ptr), int(out_ptr), int(q_rot_ptr),
                                         int(score_ptr), int(attn_out_ptr), int(total_heads), int(total_kv),
                                         int(S), int(D), int(n_levels), float(scale))


def full_compressed_attention(q_ptr: int, R_ptr: int, pk_ptr: int, km_ptr: int, ks_ptr: int, kr_ptr: int,
                              pv_ptr: int, vm_ptr: int, vs_ptr: int, vr_ptr: int, out_ptr: int, q_rot_ptr: int,
                              score_ptr: int, attn_out_ptr: int, total_heads: int, total_kv: int, S: int, D: int,
                              group_size: int, num_groups: int, scale: float) -> None:
    """polarquant_full.full_compressed_attention (csrc/polarquant_full.cu:142-186):
    group-format attention of original-space fp32 queries, output rotated
    back; device pointers as ints, asynchronous on the null stream."""
    _lib.lib().full_compressed_attention(q_ptr, R_ptr, pk_ptr, km_ptr, ks_ptr, kr_ptr, pv_ptr, vm_ptr, vs_ptr,
                                         vr_ptr, out_ptr, q_rot_ptr, score_ptr, attn_out_ptr, total_heads, total_kv,
                                         S, D, group_size, num_groups, float(scale))
