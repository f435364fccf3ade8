"""The allocation-free decode entry point (pqkv_decode_attn_noalloc) against
pqkv_decode_attn with a caller workspace, through the C ABI: the same kernels
and split plan, so the outputs must be bit-identical. Two calls in a row, the
second smaller (the shared scratch keeps the first call's contents), then a
call whose plan needs more scratch than the library holds, which is refused
before any launch."""

import numpy as np
import pytest
import torch

from oracle import oracle as O
from polarquant_kv import _lib, quantizer
from polarquant_kv.qjl import rotated_jl_matrix

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _case(B, Hq, Hkv, S, d, bits, qjl, seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    R64 = O.rotation_matrix(d, 42)
    R = torch.from_numpy(R64.astype(np.float32)).to(DEV)
    P_rot = rotated_jl_matrix(O.jl_matrix(d, d, 43), R64, DEV) if qjl else None
    k = torch.randn(B, Hkv, S, d, generator=g, device=DEV).half()
    v = torch.randn(B, Hkv, S, d, generator=g, device=DEV).half()
    kc = quantizer.compress_pq(k, R, bits, jl_rot=P_rot)
    vc = quantizer.compress_pq(v, R, bits)
    q = torch.randn(B, Hq, d, generator=g, device=DEV).half()
    return q, R, kc, vc, P_rot


def _args(q, R, kc, vc, P_rot, out):
    B, Hq, d = q.shape
    Hkv = kc.num_heads
    return [q.data_ptr(), _lib.F16, R.data_ptr(), kc.blocks.data_ptr(), vc.blocks.data_ptr(),
            kc.codebooks.data_ptr(), vc.codebooks.data_ptr(), kc.n_bits, vc.n_bits, None, None,
            _lib.ptr(kc.qjl_signs if P_rot is not None else None), _lib.ptr(P_rot), d if P_rot is not None else 0,
            B, Hq, Hkv, kc.seq_len, kc.max_seq_len, d, float(d) ** -0.5, out.data_ptr(), _lib.F32]


def _both(case):
    q, R, kc, vc, P_rot = case
    B, Hq, d = q.shape
    L = _lib.lib()
    st = _lib.stream_of(q)
    want = torch.full((B, Hq, d), float("nan"), device=DEV)
    ws = torch.empty(L.pqkv_decode_workspace_bytes(B, Hq, kc.num_heads, kc.seq_len, d), dtype=torch.uint8,
                     device=DEV)
    _lib.check(L.pqkv_decode_attn(*_args(q, R, kc, vc, P_rot, want), ws.data_ptr(), ws.numel(), st))
    got = torch.full((B, Hq, d), float("nan"), device=DEV)
    _lib.check(L.pqkv_decode_attn_noalloc(*_args(q, R, kc, vc, P_rot, got), st))
    torch.cuda.synchronize()
    return got.cpu().numpy(), want.cpu().numpy()


def test_noalloc_decode_matches_workspace_decode_twice():
    # first call: an 8B-shaped layer with QJL keys; second, smaller: a
    # different width, head dim and group size, reading scratch the first
    # call left behind
    for case in ((2, 32, 8, 5000, 128, 4, True, 1), (1, 14, 2, 700, 64, 2, False, 2)):
        print(f"noalloc decode case {case}", flush=True)
        got, want = _both(_case(*case))
        assert np.isfinite(got).all()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _scratch_bytes():
    """PQKV_NOALLOC_SCRATCH_BYTES as include/pqkv.h defines it."""
    import os
    import re
    hdr = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "pqkv.h")
    m = re.search(r"#define PQKV_NOALLOC_SCRATCH_BYTES \((\d+)u << (\d+)\)", open(hdr).read())
    return int(m.group(1)) << int(m.group(2))


def test_noalloc_refuses_a_plan_larger_than_the_scratch():
    """A shape whose rotated queries alone (B Hq d fp32) exceed the scratch
    array, on real (zeroed) device buffers of that shape: the call is refused
    before any launch, and were the refusal ever lost the kernels would read
    valid memory, not fault."""
    print("noalloc oversized plan", flush=True)
    L = _lib.lib()
    B, Hq, Hkv, S, d = 1024, 64, 8, 64, 128
    assert B * Hq * d * 4 > _scratch_bytes()
    q = torch.zeros(B, Hq, d, dtype=torch.float16, device=DEV)
    R = torch.eye(d, device=DEV)
    kc = quantizer.allocate_cache(B, Hkv, S, d, 4, DEV)
    vc = quantizer.allocate_cache(B, Hkv, S, d, 4, DEV)
    kc.seq_len = vc.seq_len = S
    out = torch.zeros(B, Hq, d, device=DEV)
    rc = L.pqkv_decode_attn_noalloc(*_args(q, R, kc, vc, None, out), _lib.stream_of(q))
    torch.cuda.synchronize()
    assert rc == _lib.ERR_WORKSPACE
    assert b"scratch" in L.pqkv_last_error()
    assert not out.any()
