"""Chunked-prefill parity over seeded random shapes: batch, kv heads, query
heads per kv head (1..8), head_dim, chunk length, chunk position, causal or
not, a cache allocated longer than the stream, and the three synthetic data
laws, against the float64 oracle on the same encoded bytes (tolerance as in
test_gpu_prefill)."""

import numpy as np
import pytest
import torch

from polarquant_kv import attention
from test_gpu_prefill import _case, _check, _oracle

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _shape(seed):
    rng = np.random.default_rng(2000 + seed)
    B = int(rng.integers(1, 3))
    Hkv = int(rng.choice([1, 2, 4]))
    G = int(rng.integers(1, 9))
    d = int(rng.choice([64, 128]))
    Sq = int(rng.integers(1, 80))
    q0 = int(rng.integers(0, 600))
    causal = bool(rng.integers(0, 2))
    S = q0 + Sq if causal else int(rng.integers(1, 700))
    S_max = S + int(rng.integers(0, 40))
    kind = str(rng.choice(["token_ln", "normal", "channel"]))
    return B, G * Hkv, Hkv, Sq, q0, S, S_max, d, causal, kind


@pytest.mark.parametrize("seed", range(12))
def test_prefill_random_shapes(seed):
    B, Hq, Hkv, Sq, q0, S, S_max, d, causal, kind = _shape(seed)
    print(f"prefill sweep seed {seed}: B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} q0={q0} S={S} S_max={S_max} d={d} "
          f"causal={causal} {kind}", flush=True)
    q, R, Rt, kc, vc = _case(B, Hq, Hkv, Sq, q0, S, d, seed=seed, kind=kind, S_max=S_max)
    out = attention.prefill_attention(torch.from_numpy(q).to(DEV), kc, vc, Rt, q_start=q0, causal=causal,
                                      out_dtype=torch.float32)
    _check(out.cpu().numpy(), _oracle(q, R, kc, vc, S, q0, causal))


def _shape_w(seed):
    rng = np.random.default_rng(2500 + seed)
    B = int(rng.integers(1, 3))
    Hkv = int(rng.choice([1, 2, 4]))
    G = int(rng.integers(1, 9))
    d = int(rng.choice([64, 128]))
    Sq = int(rng.integers(1, 64))
    q0 = int(rng.integers(0, 300))
    S = q0 + Sq
    per_head = bool(rng.integers(0, 2)) and Hkv > 1
    kb = tuple(int(x) for x in rng.choice([2, 4], Hkv)) if per_head else int(rng.choice([2, 4]))
    vb = tuple(int(x) for x in rng.choice([2, 4], Hkv)) if per_head else int(rng.choice([2, 4]))
    qjl = bool(rng.integers(0, 2))
    kind = str(rng.choice(["token_ln", "normal", "channel"]))
    return B, G * Hkv, Hkv, Sq, q0, S, d, kb, vb, qjl, kind


@pytest.mark.parametrize("seed", range(10))
def test_prefill_widths_random_shapes(seed):
    """Random shapes with 2- or 4-bit keys and values, per-head widths and the
    QJL term (causal chunks at the end of the cache)."""
    from test_gpu_prefill import _case_w, _oracle_w
    B, Hq, Hkv, Sq, q0, S, d, kb, vb, qjl, kind = _shape_w(seed)
    print(f"prefill widths sweep seed {seed}: B={B} Hq={Hq} Hkv={Hkv} Sq={Sq} q0={q0} d={d} k={kb} v={vb} "
          f"qjl={qjl} {kind}", flush=True)
    q, R, Rt, kc, vc, P, P_rot = _case_w(B, Hq, Hkv, Sq, q0, S, d, kb, vb, seed=seed, kind=kind, qjl=qjl)
    out = attention.prefill_attention(torch.from_numpy(q).to(DEV), kc, vc, Rt, q_start=q0, causal=True,
                                      out_dtype=torch.float32, jl_rot=P_rot)
    _check(out.cpu().numpy(), _oracle_w(q, R, kc, vc, S, q0, True, P=P))
