"""The reference's GPU API names on the codebook format: compress_gpu /
decompress_gpu (src/polarquant_kv_cuda/compress_kernel.py:100,
decompress_kernel.py:10), the dequantise kernel behind them, and the device
QJL helpers (qjl_kernel.py:6-70)."""

import numpy as np
import pytest
import torch

import oracle as OC
from oracle import oracle as O
from polarquant_kv import _lib, qjl, quantizer

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("d,bits", [(128, 4), (64, 4), (128, 2), (64, 2)])
def test_dequantize_bit_exact(d, bits):
    """pqkv_dequantize with fp32 output: r16 * c[code] in fp32, then the
    inverse rotation as one FMA chain per output, the C oracle's order."""
    print(f"dequantize d={d} bits={bits}", flush=True)
    rng = np.random.default_rng(d + bits)
    n = 777
    idx = rng.integers(0, 1 << bits, (n, d)).astype(np.uint8)
    r = rng.lognormal(0, 2, n).astype(np.float32)
    r[0] = 0.0
    blocks = O.pack_blocks(r, idx, bits)
    cb = O.lloyd_max_codebook(d, bits)[0]
    R = O.rotation_matrix(d, 42).astype(np.float32)
    cbp = np.zeros(16, np.float32)
    cbp[:cb.size] = cb
    bt, cbt, Rt = (torch.from_numpy(a).to(DEV) for a in (blocks, cbp, R))
    out = torch.empty(n, d, device=DEV)
    _lib.check(_lib.lib().pqkv_dequantize(bt.data_ptr(), cbt.data_ptr(), bits, Rt.data_ptr(), out.data_ptr(),
                                          _lib.F32, n, d, _lib.stream_of(out)))
    torch.cuda.synchronize()
    r16, idx2 = O.unpack_blocks(blocks, d, bits)
    xr = (r16.astype(np.float32)[:, None] * cb[idx2]).astype(np.float32)
    want = OC.c_rotate_fma(xr, R, inverse=True)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


def test_compress_gpu_decompress_gpu_round_trip():
    """compress_gpu -> decompress_gpu gives fp16 [B, H, S, d] in the original
    space, equal to the oracle's reconstruction rounded to fp16; empty input
    stays empty; large values saturate at 65504 instead of becoming inf."""
    B, H, S, d = 2, 4, 100, 128
    x = torch.from_numpy(O.synth_kv(B, H, S, d, 3, "channel")).to(DEV)
    R64 = O.rotation_matrix(d, 42)
    R = torch.from_numpy(R64.astype(np.float32)).to(DEV)
    P = O.jl_matrix(d, d, 43)
    c = quantizer.compress_gpu(x, R, 4, 32, jl_matrix=P)
    assert c.seq_len == S and c.qjl_signs is not None
    y = quantizer.decompress_gpu(c, R)
    assert y.dtype == torch.float16 and y.shape == (B, H, S, d)
    cb = O.lloyd_max_codebook(d, 4)[0]
    ref = O.inverse_rotate(O.dequantize_rotated(c.blocks.cpu().numpy(), d, cb), R64)
    got = y.float().cpu().numpy()
    np.testing.assert_allclose(got, ref, rtol=2e-3, atol=2e-3 * np.abs(ref).max() / 100 + 1e-3)
    cos = (got * x.float().cpu().numpy()).sum() / np.linalg.norm(got) / np.linalg.norm(x.float().cpu().numpy())
    assert cos > 0.99
    e = quantizer.compress_gpu(x[:, :, :0], R)
    assert e.seq_len == 0 and quantizer.decompress_gpu(e, R).shape == (B, H, 0, d)
    with pytest.raises(ValueError):
        quantizer.compress_gpu(x, R, n_bits=4, group_size=256)
    big = torch.full((1, 1, 3, d), 60000.0, device=DEV).half()
    yb = quantizer.decompress_gpu(quantizer.compress_gpu(big, R), R)
    assert torch.isfinite(yb.float()).all() and yb.float().abs().max() <= 65504


def test_decompress_mixed_and_partial():
    B, H, S, d = 1, 4, 70, 64
    x = torch.from_numpy(O.synth_kv(B, H, S, d, 5, "normal")).to(DEV)
    R = torch.from_numpy(O.rotation_matrix(d, 42).astype(np.float32)).to(DEV)
    mixed = quantizer.allocate_cache(B, H, 96, d, (4, 2, 2, 4), DEV)
    quantizer.compress_pq(x, R, cache=mixed)
    uni = quantizer.allocate_cache(B, H, 96, d, 4, DEV)
    quantizer.compress_pq(x, R, cache=uni)
    ym = quantizer.dequantize(mixed, R, torch.float32)
    yu = quantizer.dequantize(uni, R, torch.float32)
    assert ym.shape == yu.shape == (B, H, S, d)
    # the 4-bit heads of the mixed cache decode as the uniform cache's
    for h in (0, 3):
        assert torch.equal(ym[:, h], yu[:, h])
    assert not torch.equal(ym[:, 1], yu[:, 1])


def test_device_qjl_helpers():
    d, n = 128, 300
    rng = np.random.default_rng(1)
    e = rng.standard_normal((n, d)).astype(np.float32)
    e[0] = 0.0
    P = O.jl_matrix(d, d, 43)
    Pt = torch.from_numpy(P.astype(np.float32)).to(DEV)
    packed, norms = qjl.compute_signatures_gpu(torch.from_numpy(e).to(DEV), Pt)
    # the sketch sums P e in fp64 (P as given, fp32 values): signs equal the
    # fp64 product's wherever it is not within rounding of 0
    proj = e.astype(np.float64) @ P.astype(np.float32).astype(np.float64).T
    got = O.bit_unpack_lsb(packed.cpu().numpy(), d)
    clear = np.abs(proj) > 1e-9
    assert clear.mean() > 0.99
    assert np.array_equal(got[clear], (proj >= 0)[clear])
    assert got[0].all()                                        # P 0 = 0 >= 0
    np.testing.assert_allclose(norms.float().cpu().numpy(), np.linalg.norm(e, axis=1), rtol=1e-3)
    q = rng.standard_normal((n, d)).astype(np.float32)
    corr = qjl.compute_correction_gpu(torch.from_numpy(q).to(DEV), packed, norms, Pt).cpu().numpy()
    bits = O.bit_unpack_lsb(packed.cpu().numpy(), d).astype(np.float64) * 2 - 1
    want = (bits * (q.astype(np.float64) @ P.T)).sum(-1) / d
    want[0] = 0.0                      # a zero residual gets no correction (reference AC-3.5)
    assert want[1:].min() != 0.0
    np.testing.assert_allclose(corr, want, atol=1e-4)
