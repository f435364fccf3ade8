"""Decode parity over seeded random shapes: batch, kv heads, query heads per
kv head (1..10, so one or two launches per kv head), head_dim, key and value
widths, stream length (any S, not only whole tiles) and a cache allocated
longer than the stream, and the three synthetic data laws (i.i.d., per-token
norm scales, per-channel outliers), against the float64 oracle on the same encoded
bytes (tolerance of the north-star contract, as in test_gpu_decode)."""

import numpy as np
import pytest
import torch

from polarquant_kv import attention
from test_gpu_decode import _check, _oracle, _setup

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _shape(seed):
    rng = np.random.default_rng(1000 + seed)
    B = int(rng.integers(1, 4))
    Hkv = int(rng.choice([1, 2, 3, 4, 8]))
    G = int(rng.integers(1, 11))
    d = int(rng.choice([64, 128]))
    S = int(rng.integers(1, 2500))
    S_max = S + int(rng.integers(0, 50))
    kb, vb = (int(x) for x in rng.choice([2, 4], 2))
    kind = str(rng.choice(["token_ln", "normal", "channel"]))
    return B, G * Hkv, Hkv, S, S_max, d, kb, vb, kind


@pytest.mark.parametrize("seed", range(24))
def test_decode_random_shapes(seed):
    B, Hq, Hkv, S, S_max, d, kb, vb, kind = _shape(seed)
    print(f"sweep seed {seed}: B={B} Hq={Hq} Hkv={Hkv} S={S} S_max={S_max} d={d} k{kb}v{vb} {kind}", flush=True)
    q, R, Rt, kc, vc, _ = _setup(B, Hq, Hkv, S, d, kb, vb, seed=seed, S_max=S_max, kind=kind)
    out = attention.decode_attention(torch.from_numpy(q).to(DEV), kc, vc, Rt, out_dtype=torch.float32)
    _check(out.cpu().numpy(), _oracle(q, R, kc, vc, S))


@pytest.mark.parametrize("seed", range(10))
def test_decode_qjl_random_shapes(seed):
    """The same random shapes with the QJL sign sketch on the keys (m = d):
    the signs the encoder wrote and the projection P go to the oracle."""
    from oracle import oracle as O
    B, Hq, Hkv, S, S_max, d, kb, vb, kind = _shape(100 + seed)
    print(f"qjl sweep seed {seed}: B={B} Hq={Hq} Hkv={Hkv} S={S} S_max={S_max} d={d} k{kb}v{vb} {kind}", flush=True)
    q, R, Rt, kc, vc, P_rot = _setup(B, Hq, Hkv, S, d, kb, vb, seed=seed, S_max=S_max, kind=kind, qjl=True)
    out = attention.decode_attention(torch.from_numpy(q).to(DEV), kc, vc, Rt, jl_rot=P_rot, out_dtype=torch.float32)
    signs = kc.qjl_signs.cpu().numpy()[:, :, :S]
    _check(out.cpu().numpy(), _oracle(q, R, kc, vc, S, P=O.jl_matrix(d, d, 43), signs=signs))


@pytest.mark.parametrize("seed", range(10))
def test_decode_per_head_widths_random_shapes(seed):
    """Random shapes whose kv heads each take their own key and value width
    (one launch per width pair, or the paired 4/4 + 2/2 launch), with or
    without QJL."""
    from oracle import oracle as O
    from polarquant_kv import quantizer
    B, Hq, Hkv, S, S_max, d, _, _, kind = _shape(200 + seed)
    rng = np.random.default_rng(5000 + seed)
    Hkv = max(Hkv, 2)
    Hq = Hkv * int(rng.integers(1, 9))
    kw = tuple(int(x) for x in rng.choice([2, 4], Hkv))
    vw = kw if rng.integers(0, 2) else tuple(int(x) for x in rng.choice([2, 4], Hkv))
    qjl = bool(rng.integers(0, 2))
    print(f"per-head sweep seed {seed}: B={B} Hq={Hq} Hkv={Hkv} S={S} S_max={S_max} d={d} k={kw} v={vw} "
          f"qjl={qjl} {kind}", flush=True)
    k = O.synth_kv(B, Hkv, S, d, seed + 1, kind)
    v = O.synth_kv(B, Hkv, S, d, seed + 2, kind)
    q = rng.standard_normal((B, Hq, d)).astype(np.float16)
    R = O.rotation_matrix(d, 42)
    Rt = torch.from_numpy(R.astype(np.float32)).to(DEV)
    P = O.jl_matrix(d, d, 43) if qjl else None
    P_rot = torch.from_numpy((P @ R.T).astype(np.float32)).to(DEV) if qjl else None
    kc = quantizer.allocate_cache(B, Hkv, S_max, d, kw, DEV, jl_dim=d if qjl else 0)
    vc = quantizer.allocate_cache(B, Hkv, S_max, d, vw, DEV)
    quantizer.compress_pq(torch.from_numpy(k).to(DEV), Rt, cache=kc, jl_rot=P_rot)
    quantizer.compress_pq(torch.from_numpy(v).to(DEV), Rt, cache=vc)
    extra = dict(jl_rot=P_rot) if qjl else {}
    out = attention.decode_attention(torch.from_numpy(q).to(DEV), kc, vc, Rt, out_dtype=torch.float32, **extra)
    signs = kc.qjl_signs.cpu().numpy()[:, :, :S] if qjl else None
    _check(out.cpu().numpy(), _oracle(q, R, kc, vc, S, P=P, signs=signs))
