"""GPU parity of the encoders against the CPU oracle (bit-exact).

Two encoders sit behind pqkv_encode:
  * the exact encoder (PQKV_ENCODE_KERNEL=exact, and always for fp32
    input): its rotation is the reference's fp32 FMA chain, so the whole
    encode is compared bit for bit with oracle.c_rotate_fma ->
    c_quantize_rotated -> c_pack_blocks on the same inputs;
  * the matrix-core encoder (fp16 input, with or without QJL): its
    rotation has fp32-grade products with another rounding, so its quantiser
    is compared bit for bit with the oracle on the rotated values it returns
    (pqkv_encode_mfma's rot_out), and its rotation is checked against the FMA
    chain within fp32 rounding. Its QJL signs are checked against the
    oracle's projection of the residual of that rotation, up to ties."""

import numpy as np
import pytest
import torch

import oracle as OC
from oracle import oracle as O
from polarquant_kv import _lib, quantizer, rotation
from polarquant_kv.lloyd_max import padded_codebook_torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _inputs(n, d, seed, special=True):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((n, d)) * rng.lognormal(0, 1.5, (n, 1))).astype(np.float32)
    if special:
        x[0] = 0.0                                           # zero vector
        x[1] = 1e-30                                         # radius below the 1e-30 guard
        x[2] = 0.0
        x[2, 5] = 3.0                                        # one-hot
        x[3] = 1e4 * rng.standard_normal(d)                  # large
        c = O.lloyd_max_codebook(d, 4)[0]
        x[4] = c[rng.integers(0, 16, d)]                     # on the centroids
    return x


@pytest.mark.parametrize("d,bits", [(128, 4), (64, 4), (128, 2), (64, 2)])
def test_quantize_rotated_bit_exact(d, bits):
    print(f"quantize_rotated d={d} bits={bits}", flush=True)
    x = _inputs(3000, d, 1 + d + bits)
    cb = O.lloyd_max_codebook(d, bits)[0]
    blocks, radius = quantizer.quantize_rotated(torch.from_numpy(x).to(DEV), padded_codebook_torch(d, bits, DEV), bits)
    r_ref, idx_ref = OC.c_quantize_rotated(x, cb)
    torch.cuda.synchronize()
    assert np.array_equal(radius.cpu().numpy().view(np.uint32), r_ref.view(np.uint32))
    assert np.array_equal(blocks.cpu().numpy(), OC.c_pack_blocks(r_ref, idx_ref, bits))


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("inverse", [False, True])
def test_rotate_bit_exact(d, dtype, inverse):
    x = _inputs(257, d, 5, special=False)
    xt = torch.from_numpy(x).to(DEV).to(dtype)
    R = O.rotation_matrix(d, 42).astype(np.float32)
    Rt = torch.from_numpy(R).to(DEV)
    y = (rotation.inverse_rotate if inverse else rotation.rotate)(xt, Rt)
    ref = OC.c_rotate_fma(xt.float().cpu().numpy(), R, inverse=inverse)
    if dtype == torch.float32:
        assert np.array_equal(y.cpu().numpy().view(np.uint32), ref.view(np.uint32))
    else:
        assert np.array_equal(y.cpu().numpy(), ref.astype(np.float16))


def _oracle_encode(x, R32, bits):
    d = x.shape[-1]
    cb = O.lloyd_max_codebook(d, bits)[0]
    y = OC.c_rotate_fma(x.reshape(-1, d).astype(np.float32), R32)
    r, idx = OC.c_quantize_rotated(y, cb)
    return OC.c_pack_blocks(r, idx, bits), y, r, idx, cb


@pytest.mark.parametrize("d,bits", [(128, 4), (64, 4), (128, 2)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_encode_cache_bit_exact(d, bits, dtype, monkeypatch):
    print(f"encode d={d} bits={bits} dtype={dtype}", flush=True)
    monkeypatch.setenv("PQKV_ENCODE_KERNEL", "exact")
    B, H, T = 2, 3, 45
    rng = np.random.default_rng(d + bits)
    x = (rng.standard_normal((B, H, T, d)) * 2).astype(np.float32)
    xt = torch.from_numpy(x).to(DEV).to(dtype)
    R32 = O.rotation_matrix(d, 42).astype(np.float32)
    Rt = torch.from_numpy(R32).to(DEV)
    # write positions 7..51 of a 60-position cache (append at an offset)
    cache = quantizer.allocate_cache(B, H, 60, d, bits, DEV)
    quantizer.compress_pq(xt, Rt, cache=cache, start=7)
    assert cache.seq_len == 52
    want, *_ = _oracle_encode(xt.float().cpu().numpy(), R32, bits)
    got = cache.blocks.cpu().numpy()
    assert np.array_equal(got[:, :, 7:52].reshape(-1, got.shape[-1]), want)
    assert not got[:, :, :7].any() and not got[:, :, 52:].any()


def test_encode_mixed_widths_bit_exact(monkeypatch):
    monkeypatch.setenv("PQKV_ENCODE_KERNEL", "exact")
    B, H, T, d = 2, 4, 33, 128
    widths = (4, 2, 2, 4)
    rng = np.random.default_rng(3)
    x = rng.standard_normal((B, H, T, d)).astype(np.float16)
    R32 = O.rotation_matrix(d, 42).astype(np.float32)
    cache = quantizer.allocate_cache(B, H, 40, d, widths, DEV)
    quantizer.compress_pq(torch.from_numpy(x).to(DEV), torch.from_numpy(R32).to(DEV), cache=cache)
    got = cache.blocks.cpu().numpy()
    for h, bits in enumerate(widths):
        want, *_ = _oracle_encode(x[:, h].astype(np.float32), R32, bits)
        vb = O.vector_bytes(d, bits)
        off = cache.head_offset(h)
        seg = got[:, off:off + T * vb].reshape(B * T, vb)
        assert np.array_equal(seg, want), f"head {h}"


def _radius_ladder(d, seed):
    """Rows whose radii cover every branch of the exact encoders' quantiser:
    zero and below the 1e-30 guard, (1e-30, 2^-40) where directions are
    divided per coordinate, the 2^-40 edge, the normal range, squares that
    overflow to an infinite radius, and an infinite coordinate (NaN
    directions)."""
    rng = np.random.default_rng(seed)
    base = _inputs(40, d, seed)
    edge = 2.0 ** -40 / np.sqrt(d)                         # radii about 2^-40
    scales = [1e-25, 1e-20, 1e-16, 1e-14, edge, 1.1 * edge, 1e-12, 1.0, 1e15, 1e18, 1e19, 1e20]
    rows = [rng.standard_normal((3, d)) * s for s in scales]
    inf_row = rng.standard_normal((1, d))
    inf_row[0, 7] = np.inf
    return np.concatenate([base] + rows + [inf_row]).astype(np.float32)


@pytest.mark.parametrize("d,bits", [(128, 4), (64, 4), (128, 2)])
def test_encode_cache_exact_special_radii(d, bits, monkeypatch):
    print(f"exact encode radius ladder d={d} bits={bits}", flush=True)
    monkeypatch.setenv("PQKV_ENCODE_KERNEL", "exact")
    x = _radius_ladder(d, d + bits)
    n = x.shape[0]
    R32 = O.rotation_matrix(d, 42).astype(np.float32)
    cache = quantizer.allocate_cache(1, 1, n, d, bits, DEV)
    with np.errstate(invalid="ignore", over="ignore"):
        quantizer.compress_pq(torch.from_numpy(x).to(DEV).view(1, 1, n, d), torch.from_numpy(R32).to(DEV), cache=cache)
        want, *_ = _oracle_encode(x, R32, bits)
    assert np.array_equal(cache.blocks.cpu().numpy().reshape(n, -1), want)


@pytest.mark.parametrize("layout", ["paged", "misaligned", "many_steps"])
def test_encode_exact_layouts(layout, monkeypatch):
    """fp32 input on the exact encoders' other routes: paged appends (the
    register-blocked kernel's per-vector dword stores into pages), rows that
    start 4 bytes off a 16-byte boundary (the four-chain kernel, which reads
    element by element), and enough vectors that every workgroup of the
    register-blocked kernel takes several steps with a partial last one."""
    print(f"exact encode layout={layout}", flush=True)
    d, bits = 128, 4
    R32 = O.rotation_matrix(d, 42).astype(np.float32)
    Rt = torch.from_numpy(R32).to(DEV)
    if layout == "paged":
        B, H, T = 2, 3, 300
        x = _inputs(B * H * T, d, 77).reshape(B, H, T, d)
        c = quantizer.allocate_paged_cache(B, H, d, bits, DEV, page_tokens=64)
        xt = torch.from_numpy(x).to(DEV)
        for lo, hi in ((0, 1), (1, 100), (100, 300)):
            quantizer.compress_pq(xt[:, :, lo:hi].contiguous(), Rt, cache=c)
        got = c.to_contiguous().blocks.cpu().numpy().reshape(-1, 72)
    elif layout == "misaligned":
        B, H, T = 1, 2, 333
        x = _inputs(B * H * T, d, 78).reshape(B, H, T, d)
        buf = torch.zeros(x.size + 1, dtype=torch.float32, device=DEV)
        xt = buf[1:].view(B, H, T, d)
        xt.copy_(torch.from_numpy(x))
        assert xt.data_ptr() % 16 == 4
        c = quantizer.allocate_cache(B, H, T, d, bits, DEV)
        quantizer.compress_pq(xt, Rt, cache=c)
        got = c.blocks.cpu().numpy().reshape(-1, 72)
    else:
        n = 256 * 128 * 2 + 77
        x = _inputs(n, d, 79)
        c = quantizer.allocate_cache(1, 1, n, d, bits, DEV)
        quantizer.compress_pq(torch.from_numpy(x).to(DEV).view(1, 1, n, d), Rt, cache=c)
        got = c.blocks.cpu().numpy().reshape(-1, 72)
    want, *_ = _oracle_encode(x.reshape(-1, d), R32, bits)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("n", [40, 9000, 20000, 40000])
def test_encode_exact_step_sizes(n, monkeypatch):
    """The register-blocked exact encoder picks quarter-, half- or full-size
    steps by how many full-size steps a launch has (40 and 9000 vectors:
    quarter, 20000: half, 40000: full on 256 compute units); every size
    equals the oracle bit for bit."""
    print(f"exact encode step sizes n={n}", flush=True)
    monkeypatch.setenv("PQKV_ENCODE_KERNEL", "exact")
    d, bits = 128, 4
    x = _inputs(n, d, 17)
    R32 = O.rotation_matrix(d, 42).astype(np.float32)
    c = quantizer.allocate_cache(1, 1, n, d, bits, DEV)
    quantizer.compress_pq(torch.from_numpy(x).to(DEV).view(1, 1, n, d), torch.from_numpy(R32).to(DEV), cache=c)
    want, *_ = _oracle_encode(x, R32, bits)
    assert np.array_equal(c.blocks.cpu().numpy().reshape(n, -1), want)


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
@pytest.mark.parametrize("d,bits", [(128, 4), (128, 2), (64, 4), (64, 2)])
def test_encode_exact_full_steps(d, bits, dtype, monkeypatch):
    """The register-blocked exact encoder with full-size steps (4 vectors
    per thread at d = 128, 8 at d = 64; the launches above take half-size
    ones): enough vectors for several steps on every compute unit, the last
    one partial, in every input type and code width."""
    print(f"exact encode full steps d={d} bits={bits} {dtype}", flush=True)
    monkeypatch.setenv("PQKV_ENCODE_KERNEL", "exact")
    n = 256 * (32768 // d) * 2 + 77
    x = torch.from_numpy(_inputs(n, d, d + bits)).to(DEV).to(getattr(torch, dtype))
    R32 = O.rotation_matrix(d, 42).astype(np.float32)
    c = quantizer.allocate_cache(1, 1, n, d, bits, DEV)
    quantizer.compress_pq(x.view(1, 1, n, d), torch.from_numpy(R32).to(DEV), cache=c)
    want, *_ = _oracle_encode(x.float().cpu().numpy(), R32, bits)
    assert np.array_equal(c.blocks.cpu().numpy().reshape(n, -1), want)


@pytest.mark.parametrize("layout", ["contiguous", "paged", "misaligned", "qjl"])
def test_encode_bf16_bit_exact(layout):
    """bf16 input (a bf16 model's states) goes to the exact encoders as is,
    widened to fp32 on the device: the blocks equal the oracle's encode of
    x.float(), the reference's kv.float() path, bit for bit. Contiguous and
    paged rows take the register-blocked kernel, rows 2 bytes off a 16-byte
    boundary and QJL keys the four-chain kernel."""
    print(f"bf16 encode layout={layout}", flush=True)
    d, bits = 128, 4
    R = O.rotation_matrix(d, 42)
    R32 = R.astype(np.float32)
    Rt = torch.from_numpy(R32).to(DEV)
    B, H, T = 2, 2, 157
    xb = torch.from_numpy(_inputs(B * H * T, d, 91)).to(DEV).bfloat16().view(B, H, T, d)
    xf = xb.float().cpu().numpy()
    if layout == "paged":
        c = quantizer.allocate_paged_cache(B, H, d, bits, DEV, page_tokens=64)
        quantizer.compress_pq(xb[:, :, :70].contiguous(), Rt, cache=c)
        quantizer.compress_pq(xb[:, :, 70:].contiguous(), Rt, cache=c)
        got = c.to_contiguous().blocks.cpu().numpy().reshape(-1, 72)
    elif layout == "misaligned":
        buf = torch.zeros(xb.numel() + 1, dtype=torch.bfloat16, device=DEV)
        xm = buf[1:].view(B, H, T, d)
        xm.copy_(xb)
        assert xm.data_ptr() % 16 == 2
        c = quantizer.allocate_cache(B, H, T, d, bits, DEV)
        quantizer.compress_pq(xm, Rt, cache=c)
        got = c.blocks.cpu().numpy().reshape(-1, 72)
    else:
        jl = layout == "qjl"
        P_rot = (O.jl_matrix(d, d, 43) @ R.T).astype(np.float32)
        c = quantizer.allocate_cache(B, H, T, d, bits, DEV, jl_dim=d if jl else 0)
        quantizer.compress_pq(xb, Rt, cache=c, jl_rot=torch.from_numpy(P_rot).to(DEV) if jl else None)
        got = c.blocks.cpu().numpy().reshape(-1, 72)
    want, y, r, idx, cb = _oracle_encode(xf.reshape(-1, d), R32, bits)
    assert np.array_equal(got, want)
    if layout == "qjl":
        e = y.astype(np.float64) - r[:, None].astype(np.float64) * cb[idx].astype(np.float64)
        proj = e @ P_rot.astype(np.float64).T
        sg = O.bit_unpack_lsb(c.qjl_signs.cpu().numpy().reshape(-1, d // 8), d)
        want_s = O.bit_unpack_lsb(O.bit_pack_lsb(proj >= 0), d)
        # sign ties: projections within fp32 summation error of zero
        tol = 1e-5 * np.linalg.norm(e, axis=1, keepdims=True) * np.linalg.norm(P_rot, axis=1)[None]
        assert not ((sg != want_s) & (np.abs(proj) > tol)).any()
        assert (sg != want_s).mean() < 1e-3


def _qjl_check(signs, y, r, idx, cb, P_rot, d):
    """Sign m of a vector is (P_rot e)[m] >= 0 for e = y - r c[idx] of the
    FMA-chain rotation, up to ties within fp32 summation error of zero."""
    e = y.astype(np.float64) - r[:, None].astype(np.float64) * cb[idx].astype(np.float64)
    proj = e @ P_rot.astype(np.float64).T
    want = O.bit_unpack_lsb(O.bit_pack_lsb(proj >= 0), d)
    got = O.bit_unpack_lsb(signs.reshape(-1, d // 8), d)
    tol = 1e-5 * np.linalg.norm(e, axis=1, keepdims=True) * np.linalg.norm(P_rot, axis=1)[None]
    assert not ((got != want) & (np.abs(proj) > tol)).any()
    assert (got != want).mean() < 1e-3


@pytest.mark.parametrize("layout", ["contiguous", "paged", "misaligned", "many_steps"])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
@pytest.mark.parametrize("d,bits", [(128, 4), (128, 2), (64, 4)])
def test_encode_exact_qjl(d, bits, dtype, layout, monkeypatch):
    """QJL keys on the exact encoders: the register-blocked kernel's
    projection pass (contiguous, paged, many steps per workgroup) and the
    four-chain kernel (rows 2 or 4 bytes off a 16-byte boundary). The blocks
    equal the oracle's bit for bit, the signs up to ties."""
    print(f"exact QJL d={d} bits={bits} {dtype} {layout}", flush=True)
    monkeypatch.setenv("PQKV_ENCODE_KERNEL", "exact")
    R = O.rotation_matrix(d, 42)
    R32 = R.astype(np.float32)
    Rt = torch.from_numpy(R32).to(DEV)
    P_rot = (O.jl_matrix(d, d, 43) @ R.T).astype(np.float32)
    Pt = torch.from_numpy(P_rot).to(DEV)
    tdt = getattr(torch, dtype)
    B, H, T = (1, 1, 2 * 256 * 64 + 33) if layout == "many_steps" else (2, 2, 150)
    x = torch.from_numpy(_inputs(B * H * T, d, d + bits)).to(DEV).to(tdt).view(B, H, T, d)
    if layout == "paged":
        c = quantizer.allocate_paged_cache(B, H, d, bits, DEV, page_tokens=64, jl_dim=d)
        quantizer.compress_pq(x[:, :, :90].contiguous(), Rt, cache=c, jl_rot=Pt)
        quantizer.compress_pq(x[:, :, 90:].contiguous(), Rt, cache=c, jl_rot=Pt)
        cc = c.to_contiguous()
        blocks, signs = cc.blocks.cpu().numpy(), cc.qjl_signs.cpu().numpy()
    else:
        xin = x
        if layout == "misaligned":
            buf = torch.zeros(x.numel() + 1, dtype=tdt, device=DEV)
            xin = buf[1:].view(B, H, T, d)
            xin.copy_(x)
            assert xin.data_ptr() % 16 != 0
        c = quantizer.allocate_cache(B, H, T, d, bits, DEV, jl_dim=d)
        quantizer.compress_pq(xin, Rt, cache=c, jl_rot=Pt)
        blocks, signs = c.blocks.cpu().numpy(), c.qjl_signs.cpu().numpy()
    want, y, r, idx, cb = _oracle_encode(x.float().cpu().numpy().reshape(-1, d), R32, bits)
    assert np.array_equal(blocks.reshape(B * H * T, -1), want)
    _qjl_check(signs, y, r, idx, cb, P_rot, d)


def test_encode_qjl_signs(monkeypatch):
    """The exact encoder's QJL signs (fp32 FMA-chain rotation)."""
    monkeypatch.setenv("PQKV_ENCODE_KERNEL", "exact")
    B, H, T, d = 1, 2, 200, 128
    rng = np.random.default_rng(8)
    x = rng.standard_normal((B, H, T, d)).astype(np.float16)
    R = O.rotation_matrix(d, 42)
    P = O.jl_matrix(d, d, 43)
    P_rot = (P @ R.T).astype(np.float32)
    cache = quantizer.allocate_cache(B, H, T, d, 4, DEV, jl_dim=d)
    quantizer.compress_pq(torch.from_numpy(x).to(DEV), torch.from_numpy(R.astype(np.float32)).to(DEV),
                          cache=cache, jl_rot=torch.from_numpy(P_rot).to(DEV))
    blocks, y, r, idx, cb = _oracle_encode(x.astype(np.float32), R.astype(np.float32), 4)
    assert np.array_equal(cache.blocks.cpu().numpy().reshape(-1, 72), blocks)
    e = y.astype(np.float64) - r[:, None].astype(np.float64) * cb[idx].astype(np.float64)
    proj = e @ P_rot.astype(np.float64).T
    want = O.bit_unpack_lsb(O.bit_pack_lsb(proj >= 0), d)
    got = O.bit_unpack_lsb(cache.qjl_signs.cpu().numpy().reshape(-1, d // 8), d)
    # sign ties: projections within fp32 summation error of zero
    tol = 1e-5 * np.linalg.norm(e, axis=1, keepdims=True) * np.linalg.norm(P_rot, axis=1)[None]
    bad = (got != want) & (np.abs(proj) > tol)
    assert not bad.any(), int(bad.sum())
    assert (got != want).mean() < 1e-3


# ---------------------------------------------------------------------------
# matrix-core encoder
# ---------------------------------------------------------------------------

def _fp16_inputs(n, d, seed, kind):
    rng = np.random.default_rng(seed)
    if kind == "normal":
        x = rng.standard_normal((n, d))
    elif kind == "channel":
        std = np.exp(rng.standard_normal(d))
        std[rng.permutation(d)[:2]] *= 20
        x = rng.standard_normal((n, d)) * std
    else:  # special vectors among lognormal-scaled ones
        x = rng.standard_normal((n, d)) * rng.lognormal(0, 1.5, (n, 1))
        x[0] = 0.0                                           # zero vector
        x[1] = 0.0
        x[1, 3] = 6e-8                                       # fp16 subnormal, one coordinate
        x[2] = 0.0
        x[2, 5] = 3.0                                        # one-hot
        x[3] = 1e4 * rng.standard_normal(d)                  # large
        x[4] = 1.0                                           # constant
    return x.astype(np.float16)


def _encode_mfma(x16, R32, cb_t, bits, d, n_outer=1):
    n = x16.shape[0]
    vb = O.vector_bytes(d, bits)
    xt = torch.from_numpy(x16).to(DEV)
    Rt = torch.from_numpy(R32).to(DEV)
    blocks = torch.zeros(n, vb, dtype=torch.uint8, device=DEV)
    rot = torch.empty(n, d, dtype=torch.float32, device=DEV)
    rad = torch.empty(n, dtype=torch.float32, device=DEV)
    n_inner = n // n_outer
    _lib.check(_lib.lib().pqkv_encode_mfma(xt.data_ptr(), _lib.F16, n_inner * d, Rt.data_ptr(), cb_t.data_ptr(),
                                           bits, blocks.data_ptr(), n_inner * vb, n_outer, n_inner, d,
                                           rot.data_ptr(), rad.data_ptr(), _lib.stream_of(xt)))
    torch.cuda.synchronize()
    _encode_mfma.radius = rad.cpu().numpy()   # fp32 radii of the last call
    return blocks.cpu().numpy(), rot.cpu().numpy()


@pytest.mark.parametrize("d,bits", [(128, 4), (64, 4), (128, 2), (64, 2)])
@pytest.mark.parametrize("kind", ["normal", "channel", "special"])
def test_mfma_encoder_quantiser_bit_exact_on_its_rotation(d, bits, kind):
    print(f"encode_mfma d={d} bits={bits} kind={kind}", flush=True)
    x = _fp16_inputs(3001, d, d + bits, kind)              # not a multiple of the 64-vector tile
    R32 = O.rotation_matrix(d, 42).astype(np.float32)
    blocks, rot = _encode_mfma(x, R32, padded_codebook_torch(d, bits, DEV), bits, d, n_outer=3001 if kind == "normal" else 1)
    cb = O.lloyd_max_codebook(d, bits)[0]
    r_ref, idx_ref = OC.c_quantize_rotated(rot, cb)
    assert np.array_equal(blocks, OC.c_pack_blocks(r_ref, idx_ref, bits))
    assert np.array_equal(_encode_mfma.radius.view(np.uint32), r_ref.view(np.uint32))   # fp32 radii too
    if kind == "special":
        assert not blocks[0, :2].any() and r_ref[0] == 0.0  # zero vector: radius 0, code argmin |c|


@pytest.mark.parametrize("d,bits", [(128, 4), (64, 2)])
def test_mfma_rotation_within_fp32_rounding_of_fma_chain(d, bits):
    x = _fp16_inputs(4096, d, 7, "channel")
    R32 = O.rotation_matrix(d, 42).astype(np.float32)
    blocks, rot = _encode_mfma(x, R32, padded_codebook_torch(d, bits, DEV), bits, d)
    ref = OC.c_rotate_fma(x.astype(np.float32), R32)
    scale = np.abs(x.astype(np.float64)) @ np.abs(R32.astype(np.float64)).T   # sum |x_k R_jk|
    # both are fp32 sums of 128 products in different orders; dropping R's lo
    # half would leave ~2^-12 of the scale, far above this bound
    err = np.abs(rot.astype(np.float64) - ref) / scale
    assert err.max() <= 64 * 2.0 ** -24, err.max()
    cb = O.lloyd_max_codebook(d, bits)[0]
    r_ref, idx_ref = OC.c_quantize_rotated(ref, cb)
    r_got, idx_got = OC.c_quantize_rotated(rot, cb)
    assert (idx_got == idx_ref).mean() > 0.9999            # codes flip only at exact boundary cases
    assert (np.abs(r_got.astype(np.float64) / r_ref - 1) < 1e-6).all()


@pytest.mark.parametrize("n_inner", [1, 7, 64, 333])
def test_mfma_encoder_strided_rows(n_inner):
    """Rows with gaps in x and in the blocks (no flattening): the per-vector
    row split must land every vector where the contiguous encode puts it."""
    d, bits, n_outer = 128, 4, 37
    print(f"encode_mfma strided rows n_inner={n_inner}", flush=True)
    vb = O.vector_bytes(d, bits)
    x = _fp16_inputs(n_outer * n_inner, d, n_inner, "channel")
    R32 = O.rotation_matrix(d, 42).astype(np.float32)
    cb_t = padded_codebook_torch(d, bits, DEV)
    want, _ = _encode_mfma(x, R32, cb_t, bits, d)
    xs, bs = n_inner + 3, n_inner + 5                      # row strides in vectors
    xpad = np.zeros((n_outer, xs, d), np.float16)
    xpad[:, :n_inner] = x.reshape(n_outer, n_inner, d)
    xt = torch.from_numpy(xpad).to(DEV)
    Rt = torch.from_numpy(R32).to(DEV)
    blocks = torch.full((n_outer, bs, vb), 0xAB, dtype=torch.uint8, device=DEV)
    _lib.check(_lib.lib().pqkv_encode_mfma(xt.data_ptr(), _lib.F16, xs * d, Rt.data_ptr(), cb_t.data_ptr(), bits,
                                           blocks.data_ptr(), bs * vb, n_outer, n_inner, d, None, None,
                                           _lib.stream_of(xt)))
    torch.cuda.synchronize()
    got = blocks.cpu().numpy()
    assert np.array_equal(got[:, :n_inner].reshape(-1, vb), want)
    assert (got[:, n_inner:] == 0xAB).all()                 # gaps untouched


def test_mfma_encoder_nonfinite_rows():
    """inf / NaN coordinates take the per-coordinate division form for their
    tile; the quantiser still matches the reference's on the rotated values."""
    d, bits = 128, 4
    x = _fp16_inputs(200, d, 11, "normal")
    x[5, 7] = np.inf
    x[20, 0] = -np.inf
    x[21, :] = np.inf
    x[40, 9] = np.nan
    x[70, 3], x[70, 4] = np.inf, -np.inf
    R32 = O.rotation_matrix(d, 42).astype(np.float32)
    blocks, rot = _encode_mfma(x, R32, padded_codebook_torch(d, bits, DEV), bits, d)
    cb = O.lloyd_max_codebook(d, bits)[0]
    r_ref, idx_ref = OC.c_quantize_rotated(rot, cb)
    want = OC.c_pack_blocks(r_ref, idx_ref, bits)
    codes = np.concatenate([np.arange(2, 18), np.arange(20, 36), np.arange(38, 54), np.arange(56, 72)])
    assert np.array_equal(blocks[:, codes], want[:, codes])  # index bytes
    rad_got = blocks[:, [0, 1, 18, 19, 36, 37, 54, 55]].copy().view(np.float16).astype(np.float32)
    rad_want = want[:, [0, 1, 18, 19, 36, 37, 54, 55]].copy().view(np.float16).astype(np.float32)
    assert np.array_equal(np.isnan(rad_got), np.isnan(rad_want))
    ok = ~np.isnan(rad_want)
    assert np.array_equal(rad_got[ok], rad_want[ok])
    assert np.isnan(rot[40]).any() and not np.isfinite(rad_want[40]).all()


def test_mfma_encoder_unsorted_codebook_uses_the_scan():
    d, bits = 128, 4
    x = _fp16_inputs(700, d, 3, "normal")
    R32 = O.rotation_matrix(d, 42).astype(np.float32)
    cb = O.lloyd_max_codebook(d, bits)[0]
    perm = np.random.default_rng(0).permutation(16)
    cbp = cb[perm].astype(np.float32)
    blocks, rot = _encode_mfma(x, R32, torch.from_numpy(cbp).to(DEV), bits, d)
    r_ref, idx_ref = OC.c_quantize_rotated(rot, cbp)
    assert np.array_equal(blocks, OC.c_pack_blocks(r_ref, idx_ref, bits))


def test_compress_pq_fp16_takes_the_mfma_encoder(monkeypatch):
    B, H, T, d = 2, 3, 150, 128
    x = _fp16_inputs(B * H * T, d, 9, "normal").reshape(B, H, T, d)
    R32 = O.rotation_matrix(d, 42).astype(np.float32)
    Rt = torch.from_numpy(R32).to(DEV)
    cache = quantizer.allocate_cache(B, H, 160, d, 4, DEV)
    quantizer.compress_pq(torch.from_numpy(x).to(DEV), Rt, cache=cache)
    got = cache.blocks.cpu().numpy()[:, :, :T].reshape(-1, 72)
    want, _ = _encode_mfma(x.reshape(-1, d), R32, padded_codebook_torch(d, 4, DEV), 4, d)
    assert np.array_equal(got, want)
    monkeypatch.setenv("PQKV_ENCODE_KERNEL", "exact")
    quantizer.compress_pq(torch.from_numpy(x).to(DEV), Rt, cache=cache, start=0)
    want_exact, *_ = _oracle_encode(x.astype(np.float32), R32, 4)
    assert np.array_equal(cache.blocks.cpu().numpy()[:, :, :T].reshape(-1, 72), want_exact)


@pytest.mark.parametrize("d,bits", [(128, 4), (64, 4), (128, 2)])
@pytest.mark.parametrize("layout", ["strided", "contiguous"])
def test_mfma_encoder_qjl_signs(d, bits, layout):
    """QJL keys on the matrix-core encoder: the blocks are the non-QJL
    encoder's bit for bit (same rotation, same quantiser), and sign m of a
    vector is (P_rot e)[m] >= 0 for e = y - r c[code] of that rotation (y, r
    from pqkv_encode_mfma's rot_out / radius_out), up to projections within
    fp32 summation error of zero."""
    print(f"encode_mfma qjl d={d} bits={bits} {layout}", flush=True)
    B, H, T = 2, 3, 333
    S_max = T if layout == "contiguous" else T + 11
    x = _fp16_inputs(B * H * T, d, 100 + d + bits, "special").reshape(B, H, T, d)
    R32 = O.rotation_matrix(d, 42).astype(np.float32)
    P_rot = (O.jl_matrix(d, d, 43) @ R32.astype(np.float64).T).astype(np.float32)
    cache = quantizer.allocate_cache(B, H, S_max, d, bits, DEV, jl_dim=d)
    quantizer.compress_pq(torch.from_numpy(x).to(DEV), torch.from_numpy(R32).to(DEV), cache=cache,
                          jl_rot=torch.from_numpy(P_rot).to(DEV))
    torch.cuda.synchronize()
    vb = O.vector_bytes(d, bits)
    got_blocks = cache.blocks.cpu().numpy()[:, :, :T].reshape(-1, vb)
    want_blocks, rot = _encode_mfma(x.reshape(-1, d), R32, padded_codebook_torch(d, bits, DEV), bits, d)
    assert np.array_equal(got_blocks, want_blocks)
    cb = O.lloyd_max_codebook(d, bits)[0]
    r, idx = OC.c_quantize_rotated(rot, cb)
    assert np.array_equal(_encode_mfma.radius.view(np.uint32), r.view(np.uint32))
    e = rot.astype(np.float64) - r[:, None].astype(np.float64) * cb[idx].astype(np.float64)
    proj = e @ P_rot.astype(np.float64).T
    want = proj >= 0
    got = O.bit_unpack_lsb(cache.qjl_signs.cpu().numpy()[:, :, :T].reshape(-1, d // 8), d)
    tol = 1e-5 * np.linalg.norm(e, axis=1, keepdims=True) * np.linalg.norm(P_rot, axis=1)[None]
    bad = (got != want) & (np.abs(proj) > tol)
    assert not bad.any(), int(bad.sum())
    assert (got != want).mean() < 1e-3
    assert got[0].all()                                       # zero vector: e = 0, every projection >= 0
    if S_max > T:
        assert not cache.qjl_signs[:, :, T:].any().item()     # padding positions untouched
