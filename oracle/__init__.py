"""CPU oracle for the PolarQuant-KV hot path (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker or the timed CPU baseline.
"""

import ctypes
import os
import subprocess

import numpy as np

from . import oracle  # noqa: F401

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def build() -> str:
    """Compile oracle/libpq_oracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return os.path.join(_HERE, "libpq_oracle.so")


def clib():
    """ctypes handle on the C restatement (built on first use if absent)."""
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "libpq_oracle.so")
        if not os.path.exists(path):
            build()
        lib = ctypes.CDLL(path)
        lib.pq_oracle_quantize_rotated.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
            ctypes.c_void_p, ctypes.c_long, ctypes.c_int]
        lib.pq_oracle_pack_blocks.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
            ctypes.c_long, ctypes.c_int]
        lib.pq_oracle_rotate_fma.argtypes = [
            ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_long, ctypes.c_int, ctypes.c_int]
        _LIB = lib
    return _LIB


def c_quantize_rotated(x_rot, centroids):
    x = np.ascontiguousarray(x_rot, np.float32)
    cb = np.ascontiguousarray(centroids, np.float32)
    n, d = x.shape
    r = np.empty(n, np.float32)
    idx = np.empty((n, d), np.uint8)
    rc = clib().pq_oracle_quantize_rotated(x.ctypes.data, cb.ctypes.data, cb.shape[0],
                                           r.ctypes.data, idx.ctypes.data, n, d)
    if rc != 0:
        raise ValueError(f"pq_oracle_quantize_rotated rc={rc}")
    return r, idx


def c_pack_blocks(radius, idx, n_bits=4):
    r = np.ascontiguousarray(radius, np.float32)
    q = np.ascontiguousarray(idx, np.uint8)
    n, d = q.shape
    bb = 18 if n_bits == 4 else 10
    out = np.empty((n, d // 32 * bb), np.uint8)
    rc = clib().pq_oracle_pack_blocks(r.ctypes.data, q.ctypes.data, n_bits,
                                      out.ctypes.data, n, d)
    if rc != 0:
        raise ValueError(f"pq_oracle_pack_blocks rc={rc}")
    return out


def c_rotate_fma(x, R, inverse=False):
    """fp32 FMA-chain rotation (bit-exact model of the reference kernels)."""
    xv = np.ascontiguousarray(x, np.float32)
    Rf = np.ascontiguousarray(R, np.float32)
    n, d = xv.shape
    y = np.empty((n, d), np.float32)
    rc = clib().pq_oracle_rotate_fma(xv.ctypes.data, Rf.ctypes.data, y.ctypes.data, n, d, int(inverse))
    if rc != 0:
        raise ValueError(f"pq_oracle_rotate_fma rc={rc}")
    return y
