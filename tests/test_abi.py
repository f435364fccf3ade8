"""The C ABI (include/pqkv.h) on a machine without a GPU: the library loads,
exports every declared function, and rejects bad arguments in host code
before any HIP call. No compute call is made here."""

import ctypes
import os
import re

import numpy as np
import pytest

from conftest import ROOT
from polarquant_kv import _lib

HEADER = os.path.join(ROOT, "include", "pqkv.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b([a-z_][a-z0-9_]*)\s*\(", text)
    keywords = {"if", "sizeof", "defined", "return"}
    return sorted({n for n in names if n not in keywords and (n.startswith(("pqkv_", "polarquant_", "turboquant_"))
                                                                or n == "full_compressed_attention")})


def test_header_declares_the_surface():
    names = declared_functions()
    assert "pqkv_decode_attn" in names and "polarquant_fused_attention_cuda_c" in names
    assert set(names) == set(_lib.SIGNATURES), "ctypes table and header disagree"


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing


def test_layout_helpers():
    L = _lib.lib()
    assert L.pqkv_block_bytes(4) == 18 and L.pqkv_block_bytes(2) == 10 and L.pqkv_block_bytes(3) < 0
    assert L.pqkv_vector_bytes(128, 4) == 72 and L.pqkv_vector_bytes(64, 4) == 36
    assert L.pqkv_vector_bytes(128, 2) == 40 and L.pqkv_vector_bytes(100, 4) < 0
    assert L.pqkv_version() >= 1
    assert L.pqkv_status_string(_lib.ERR_WORKSPACE) == b"workspace too small"


@pytest.mark.parametrize("d,bits", [(64, 2), (64, 3), (64, 4), (128, 2), (128, 3), (128, 4)])
def test_host_codebook_matches_reference_golden(d, bits, golden_codebooks):
    c = np.zeros(1 << bits, np.float32)
    b = np.zeros((1 << bits) + 1, np.float32)
    _lib.check(_lib.lib().pqkv_lloyd_max_codebook(d, bits, 300, 50000, c.ctypes.data, b.ctypes.data))
    gc, gb = golden_codebooks[f"d{d}_b{bits}"]
    assert np.array_equal(c, gc)
    # The middle boundary is (c[L/2-1] + c[L/2]) / 2 of the pre-final
    # centroids, a cancellation to ~1e-17 whose last bits follow the summation
    # rounding of scipy's pdf; the boundaries are not used for quantisation.
    np.testing.assert_allclose(b, gb, rtol=0, atol=1e-15)


FAKE = 0x1000  # never dereferenced: every call below fails validation first


def _status(rc, expect):
    assert rc == expect, _lib.lib().pqkv_last_error()
    assert _lib.lib().pqkv_last_error()


def test_validation_rejects_before_touching_the_gpu():
    L = _lib.lib()
    _status(L.pqkv_rotate(FAKE, 0, FAKE, FAKE, 0, 10, 96, 0, None), _lib.ERR_UNSUPPORTED)
    _status(L.pqkv_rotate(FAKE, 5, FAKE, FAKE, 0, 10, 128, 0, None), _lib.ERR_UNSUPPORTED)
    _status(L.pqkv_rotate(FAKE, 0, FAKE, FAKE, 0, -1, 128, 0, None), _lib.ERR_INVALID)
    _status(L.pqkv_quantize_rotated(FAKE, FAKE, 3, FAKE, None, 4, 128, None), _lib.ERR_UNSUPPORTED)
    _status(L.pqkv_quantize_rotated(None, FAKE, 4, FAKE, None, 4, 128, None), _lib.ERR_INVALID)
    _status(L.pqkv_encode(FAKE, 1, 128, FAKE, FAKE, 4, FAKE, 72, -1, 1, 128, None, 0, None, 0, None),
            _lib.ERR_INVALID)
    # QJL needs both the projection and the output, and m == d
    _status(L.pqkv_encode(FAKE, 1, 128, FAKE, FAKE, 4, FAKE, 72, 1, 1, 128, FAKE, 128, None, 0, None),
            _lib.ERR_INVALID)
    _status(L.pqkv_encode(FAKE, 1, 128, FAKE, FAKE, 4, FAKE, 72, 1, 1, 128, FAKE, 64, FAKE, 16, None),
            _lib.ERR_UNSUPPORTED)
    # overlapping outer strides
    _status(L.pqkv_encode(FAKE, 1, 10, FAKE, FAKE, 4, FAKE, 72, 2, 4, 128, None, 0, None, 0, None),
            _lib.ERR_INVALID)


def _decode(**kw):
    args = dict(q=FAKE, qt=1, R=FAKE, k=FAKE, v=FAKE, kcb=FAKE, vcb=FAKE, kb=4, vb=4, khb=None, vhb=None,
                qjl=None, p=None, m=0, B=1, Hq=8, Hkv=2, S=16, S_max=16, d=128, scale=0.088, out=FAKE, ot=1,
                ws=FAKE, wsb=1 << 20)
    args.update(kw)
    a = args
    return _lib.lib().pqkv_decode_attn(a["q"], a["qt"], a["R"], a["k"], a["v"], a["kcb"], a["vcb"], a["kb"],
                                       a["vb"], a["khb"], a["vhb"], a["qjl"], a["p"], a["m"], a["B"], a["Hq"],
                                       a["Hkv"], a["S"], a["S_max"], a["d"], a["scale"], a["out"], a["ot"],
                                       a["ws"], a["wsb"], None)


def test_decode_validation():
    _status(_decode(Hq=6, Hkv=4), _lib.ERR_INVALID)            # Hq not a multiple of Hkv
    _status(_decode(Hq=32, Hkv=2, wsb=16), _lib.ERR_WORKSPACE)  # a group of 16 passes validation
    _status(_decode(d=96), _lib.ERR_UNSUPPORTED)
    _status(_decode(kb=3), _lib.ERR_UNSUPPORTED)
    _status(_decode(S=20, S_max=16), _lib.ERR_INVALID)
    _status(_decode(scale=0.0), _lib.ERR_INVALID)
    _status(_decode(qjl=FAKE), _lib.ERR_INVALID)               # signs without projection
    _status(_decode(qjl=FAKE, p=FAKE, m=64), _lib.ERR_UNSUPPORTED)
    _status(_decode(wsb=16), _lib.ERR_WORKSPACE)
    _status(_decode(ws=None), _lib.ERR_WORKSPACE)
    bits = _lib.int_array([4, 3])
    _status(_decode(khb=bits), _lib.ERR_UNSUPPORTED)
    need = _lib.lib().pqkv_decode_workspace_bytes(8, 32, 8, 32768, 128)
    assert need >= 8 * 32 * 128 * 2


def _prefill(**kw):
    a = dict(q=FAKE, qt=1, R=FAKE, k=FAKE, v=FAKE, kcb=FAKE, vcb=FAKE, kb=4, vb=4, khb=None, vhb=None, qjl=None,
             p=None, m=0, B=1, Hq=8, Hkv=2, Sq=16, q0=48, S=64, S_max=64, d=128, scale=0.088, causal=1, out=FAKE,
             ot=1, ws=FAKE, wsb=1 << 24)
    a.update(kw)
    return _lib.lib().pqkv_prefill_attn(a["q"], a["qt"], a["R"], a["k"], a["v"], a["kcb"], a["vcb"], a["kb"],
                                        a["vb"], a["khb"], a["vhb"], a["qjl"], a["p"], a["m"], a["B"], a["Hq"],
                                        a["Hkv"], a["Sq"], a["q0"], a["S"], a["S_max"], a["d"], a["scale"],
                                        a["causal"], a["out"], a["ot"], a["ws"], a["wsb"], None)


def test_prefill_validation():
    _status(_prefill(Hq=6, Hkv=4), _lib.ERR_INVALID)
    _status(_prefill(q0=60), _lib.ERR_INVALID)                 # causal queries past the cache
    _status(_prefill(q0=-1), _lib.ERR_INVALID)
    _status(_prefill(S=80), _lib.ERR_INVALID)                  # S > S_max
    _status(_prefill(d=96), _lib.ERR_UNSUPPORTED)
    _status(_prefill(kb=3), _lib.ERR_UNSUPPORTED)              # 2- and 4-bit codes
    _status(_prefill(qjl=FAKE), _lib.ERR_INVALID)              # signs without projection
    _status(_prefill(qjl=FAKE, p=FAKE, m=64), _lib.ERR_UNSUPPORTED)
    _status(_prefill(khb=_lib.int_array([4, 3])), _lib.ERR_UNSUPPORTED)
    _status(_prefill(kb=2, vb=2, khb=_lib.int_array([4, 2]), wsb=16), _lib.ERR_WORKSPACE)
    _status(_prefill(scale=-1.0), _lib.ERR_INVALID)
    _status(_prefill(R=FAKE + 4), _lib.ERR_INVALID)            # R alignment
    _status(_prefill(wsb=1024), _lib.ERR_WORKSPACE)
    need = _lib.lib().pqkv_prefill_workspace_bytes(1, 64, 8, 2048, 133120, 128)
    assert need == 3 * 64 * 2048 * 128 * 4
    assert _prefill(Sq=0) == 0                                 # nothing to do


def test_zero_sized_calls_are_no_ops():
    L = _lib.lib()
    assert L.pqkv_rotate(None, 0, None, None, 0, 0, 128, 0, None) == 0
    assert L.pqkv_quantize_rotated(None, None, 4, None, None, 0, 64, None) == 0
    assert L.pqkv_encode(None, 0, 0, None, None, 4, None, 0, 0, 5, 128, None, 0, None, 0, None) == 0
    assert L.pqkv_soa_to_blocks(None, None, None, 0, 128, None) == 0


def test_paged_validation():
    """The paged entry points check the page size, the table width and the
    widths in host code (fake pointers never reach a launch)."""
    L = _lib.lib()
    # pqkv_encode_paged(x, dt, xs, R, cb, bits, pages, P, max_pages, start, streams, tokens, d, p, m, qjl, stream)
    def enc(**k):
        a = dict(x=FAKE, dt=1, xs=1280, R=FAKE, cb=FAKE, bits=4, pages=FAKE, P=64, mp=4, start=0, ns=2, nt=10,
                 d=128, p=None, m=0, qjl=None)
        a.update(k)
        return L.pqkv_encode_paged(a["x"], a["dt"], a["xs"], a["R"], a["cb"], a["bits"], a["pages"], a["P"],
                                   a["mp"], a["start"], a["ns"], a["nt"], a["d"], a["p"], a["m"], a["qjl"], None)
    _status(enc(P=48), _lib.ERR_INVALID)                       # not a power of two
    _status(enc(P=32), _lib.ERR_INVALID)                       # below one 64-token chunk
    _status(enc(P=1 << 17), _lib.ERR_INVALID)
    _status(enc(mp=0), _lib.ERR_INVALID)
    _status(enc(start=250, mp=4), _lib.ERR_INVALID)            # 260 positions need 5 pages of 64
    _status(enc(start=-1), _lib.ERR_INVALID)
    _status(enc(bits=3), _lib.ERR_UNSUPPORTED)
    _status(enc(xs=100), _lib.ERR_INVALID)                     # rows overlap
    _status(enc(p=FAKE, m=128), _lib.ERR_INVALID)              # projection without sign pages
    assert enc(nt=0, start=0) == 0                             # nothing to write

    def dec(**k):
        a = dict(q=FAKE, qt=1, R=FAKE, kp=FAKE, vp=FAKE, P=64, mp=4, kcb=FAKE, vcb=FAKE, bits=4, qjl=None, p=None,
                 m=0, B=1, Hq=8, Hkv=2, S=200, d=128, scale=0.088, out=FAKE, ot=1, ws=FAKE, wsb=1 << 20)
        a.update(k)
        return L.pqkv_decode_attn_paged(a["q"], a["qt"], a["R"], a["kp"], a["vp"], a["P"], a["mp"], a["kcb"],
                                        a["vcb"], a["bits"], a["qjl"], a["p"], a["m"], a["B"], a["Hq"], a["Hkv"],
                                        a["S"], a["d"], a["scale"], a["out"], a["ot"], a["ws"], a["wsb"], None)
    _status(dec(P=100), _lib.ERR_INVALID)
    _status(dec(S=300), _lib.ERR_INVALID)                      # 300 positions need 5 pages of 64
    _status(dec(bits=3), _lib.ERR_UNSUPPORTED)
    _status(dec(qjl=FAKE), _lib.ERR_INVALID)                   # sign pages without projection
    _status(dec(kp=None), _lib.ERR_INVALID)
    _status(dec(wsb=16), _lib.ERR_WORKSPACE)
    _status(dec(Hq=6, Hkv=4), _lib.ERR_INVALID)

    def pre(**k):
        a = dict(q=FAKE, qt=1, R=FAKE, kp=FAKE, vp=FAKE, P=64, mp=4, kcb=FAKE, vcb=FAKE, bits=4, qjl=None, p=None,
                 m=0, B=1, Hq=8, Hkv=2, Sq=16, q0=184, S=200, d=128, scale=0.088, causal=1, out=FAKE, ot=1,
                 ws=FAKE, wsb=1 << 24)
        a.update(k)
        return L.pqkv_prefill_attn_paged(a["q"], a["qt"], a["R"], a["kp"], a["vp"], a["P"], a["mp"], a["kcb"],
                                         a["vcb"], a["bits"], a["qjl"], a["p"], a["m"], a["B"], a["Hq"], a["Hkv"],
                                         a["Sq"], a["q0"], a["S"], a["d"], a["scale"], a["causal"], a["out"],
                                         a["ot"], a["ws"], a["wsb"], None)
    _status(pre(P=96), _lib.ERR_INVALID)
    _status(pre(S=257, q0=241), _lib.ERR_INVALID)              # table too narrow
    _status(pre(q0=190), _lib.ERR_INVALID)                     # causal queries past the cache
    _status(pre(bits=3), _lib.ERR_UNSUPPORTED)
    _status(pre(vp=None), _lib.ERR_INVALID)
    _status(pre(wsb=1024), _lib.ERR_WORKSPACE)
    assert pre(Sq=0) == 0
