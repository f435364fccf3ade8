"""Mixed-precision policies (polarquant_kv.policies, the reference's
token_importance.py / adaptive_bitwidth.py / cross_layer.py): host logic,
checked against values worked out by hand from the reference's rules."""

import pytest
import torch

from polarquant_kv import policies


def test_token_bitwidths_sink_and_window():
    b = policies.compute_token_bitwidths(100, sink_size=4, window_size=64)
    assert b.dtype == torch.int32 and b.shape == (100,)
    assert (b[:4] == 4).all() and (b[4:36] == 2).all() and (b[36:] == 4).all()
    assert (policies.compute_token_bitwidths(50) == 4).all()          # 50 <= 4 + 64: all high
    assert (policies.compute_token_bitwidths(3) == 4).all()
    assert policies.compute_token_bitwidths(0).numel() == 0
    low = policies.compute_token_bitwidths(10, sink_size=2, window_size=3, high_bits=8, low_bits=3)
    assert low.tolist() == [8, 8, 3, 3, 3, 3, 3, 8, 8, 8]
    # the reference's bits[-0:] marks the whole sequence when window_size = 0
    assert (policies.compute_token_bitwidths(10, sink_size=4, window_size=0) == 4).all()


def test_mixed_compression_ratio_estimate():
    # 1000 tokens: 4 sinks + 64 window at 4 bits, 932 at 2 bits
    avg = (68 * 4 + 932 * 2) / 1000
    assert abs(policies.estimate_mixed_compression_ratio(1000) - 16.0 / avg) < 1e-6


@pytest.mark.parametrize("L,want", [
    (1, [4]), (2, [4, 4]),
    (3, [3, 2, 4]),                       # [4, 2, 4] -> layer 0 loses a bit (layer 1 is at min)
    (4, [4, 2, 2, 4]),                    # round(2.667) = 3 -> [4, 3, 3, 4] -> the two middle ones drop
    (5, [4, 2, 2, 3, 4]),                 # [4, 3, 2, 3, 4] -> layer 1 drops, mean 3.0
    (9, [4, 4, 2, 2, 2, 2, 3, 4, 4]),     # 3.5 -> 4 and 2.5 -> 2 (half to even); layer 2 drops
])
def test_layer_bitwidths_u_shape(L, want):
    assert policies.compute_layer_bitwidths(L) == want


def test_layer_bitwidths_target_met_or_all_min():
    for L in range(3, 41):
        w = policies.compute_layer_bitwidths(L, target_avg_bits=2.5)
        assert sum(w) / L <= 2.5 + 1e-12 or all(x == 2 for x in w[1:-1])
        assert all(2 <= x <= 4 for x in w)
        assert w[0] >= w[L // 2] and w[-1] >= w[L // 2]


def test_adaptive_compression_ratio_estimate():
    # bits + 4/128*32 = bits + 1 per value: (5 + 3) / 2 = 4 -> 16 / 4
    assert policies.estimate_adaptive_compression_ratio([4, 2], head_dim=128) == 4.0


def test_cross_layer_round_trip_and_metrics():
    g = torch.Generator().manual_seed(0)
    layers = [torch.randn(2, 3, 5, 16, generator=g) for _ in range(4)]
    enc = policies.differential_encode(layers)
    assert torch.equal(enc[0], layers[0]) and torch.allclose(enc[2], layers[2] - layers[1])
    dec = policies.differential_decode(enc)
    for a, b in zip(dec, layers):
        assert torch.allclose(a, b, atol=1e-6)
    same = policies.measure_cross_layer_similarity([layers[0], layers[0].clone()])
    assert same[0]["layer"] == 1 and abs(same[0]["cosine_similarity"] - 1) < 1e-6
    assert same[0]["diff_norm_ratio"] == 0.0
    neg = policies.measure_cross_layer_similarity([layers[0], -layers[0]])
    assert abs(neg[0]["cosine_similarity"] + 1) < 1e-6 and abs(neg[0]["diff_norm_ratio"] - 2) < 1e-5
    assert abs(policies.estimate_differential_gain(10, 0.4) - 1 / (1 - 0.6 * 0.9 * 0.3)) < 1e-12
    assert policies.estimate_differential_gain(1) == 1.0


def test_token_mixed_cache_refuses_cpu_tensors():
    k = torch.zeros(1, 1, 8, 64)
    with pytest.raises(ValueError, match="no CPU fallback"):
        policies.TokenMixedCache.from_kv(k, k, torch.eye(64), policies.compute_token_bitwidths(8))
