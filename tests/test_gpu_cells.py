"""The encoders' centroid table at the places where it could differ from the
reference's scan: directions one ulp below, at and above every switch point
(the smallest fp32 value the first-minimum scan of flash_turboquant.cu:162-170
maps to the next index) and at every cell boundary of the table, for
codebooks whose switch points the table build finds by each of its routes
(the midpoint probe, the probe half an ulp from zero for a pair symmetric
about zero, the 16-ary search) and for codebooks it refuses.

The directions are planted through the SoA encoder (polarquant_compress_cuda_c)
with R = I, so each rotated coordinate is the input coordinate itself, and
the oracle is the C restatement of the reference's radius tree and scan."""

import numpy as np
import pytest
import torch

import oracle as OC
from oracle import oracle as O
from polarquant_kv import _lib, quantizer

DEV = "cuda:0"
D = 128
PLANT = 8            # planted coordinates per vector; the rest set the radius


def _scan(dv, cb):
    """First minimum of fp32 |d - c_k| over the codebook (the reference scan)."""
    dist = np.abs(dv[:, None].astype(np.float32) - cb[None, :].astype(np.float32))
    return np.argmin(dist, axis=1)


def _key(f):
    i = np.float32(f).view(np.int32).astype(np.int64)
    return i if i >= 0 else -(i & 0x7FFFFFFF)


def _kfloat(k):
    k = int(k)
    return np.array([k if k >= 0 else (-k) | 0x80000000], np.uint32).view(np.float32)[0]


def _switch_points(cb):
    """theta_i: the smallest fp32 d in (c_i, c_{i+1}] that the scan maps to
    i + 1 or more, by bisection over fp32 values (the scan is monotone in d
    for an increasing codebook)."""
    out = []
    for i in range(len(cb) - 1):
        lo, hi = _key(cb[i]), _key(cb[i + 1])
        assert _scan(np.array([_kfloat(lo)], np.float32), cb)[0] <= i
        assert _scan(np.array([_kfloat(hi)], np.float32), cb)[0] >= i + 1
        while hi - lo > 1:
            mid = (lo + hi) // 2
            if _scan(np.array([_kfloat(mid)], np.float32), cb)[0] >= i + 1:
                hi = mid
            else:
                lo = mid
        out.append(hi)
    return out


def _targets(cb):
    """Directions: each switch point and its fp32 neighbours, each cell
    boundary (k + 1/2) / 512 of the table and its neighbours, 0 and +-1."""
    keys = set()
    for k in _switch_points(cb):
        keys.update((k - 1, k, k + 1))
    for b in range(-512, 512):
        k = _key(np.float32((2 * b + 1) / 1024.0))
        keys.update((k - 1, k, k + 1))
    keys.update((0, _key(1.0), _key(-1.0)))
    return np.array([_kfloat(k) for k in sorted(keys)], np.float32)


def _radius(x):
    return OC.c_quantize_rotated(x, np.zeros(2, np.float32))[0]


def _plant(targets, seed):
    """Vectors whose planted coordinates have RN(x_j / r) at the targets, r
    being the reference tree's radius of the whole vector. A target above 1/2
    in magnitude gets a vector of its own (the rest zero for +-1); smaller
    ones share one, up to PLANT with sum tau^2 <= 1/2. The other coordinates
    are random; the planted values are re-set from the measured radius until
    it stops changing, then a lone target still missed is searched for within
    a few fp32 steps of its value (each step re-measuring the radius). The
    random coordinates are scaled so that the exact radius is 1."""
    rng = np.random.default_rng(seed)
    groups, cur, acc = [], [], 0.0
    for i in np.argsort(-np.abs(targets), kind="stable"):
        t2 = float(targets[i]) ** 2
        if t2 > 0.25:
            groups.append([i])
            continue
        if cur and (len(cur) == PLANT or acc + t2 > 0.5):
            groups.append(cur)
            cur, acc = [], 0.0
        cur.append(i)
        acc += t2
    if cur:
        groups.append(cur)
    n = len(groups)
    slot = np.full((n, PLANT), -1)
    for v, g in enumerate(groups):
        slot[v, :len(g)] = g
    tau = np.where(slot >= 0, targets[np.maximum(slot, 0)], np.float32(0)).astype(np.float32)
    # the filler's norm makes the exact radius 1: the planted values start
    # at their targets and the fixed point is a few roundings away
    f = rng.standard_normal((n, D - PLANT))
    rest = np.maximum(1.0 - (tau.astype(np.float64) ** 2).sum(axis=1), 0.0)
    f *= np.sqrt(rest / (f ** 2).sum(axis=1))[:, None]
    x = np.concatenate([tau, f.astype(np.float32)], axis=1)
    r = np.ones(n, np.float32)
    for _ in range(200):
        x[:, :PLANT] = tau * r[:, None]
        r_new = _radius(x)
        done = np.array_equal(r_new.view(np.uint32), r.view(np.uint32))
        r = r_new
        if done:
            break
    for v in np.flatnonzero(((x[:, :PLANT] / r[:, None]) != tau).any(axis=1) & (slot[:, 1] < 0)):
        cand = np.repeat(x[v:v + 1], 81, axis=0)
        t0 = cand[0, 0]
        for k in range(81):
            t = t0
            for _ in range(abs(k - 40)):
                t = np.nextafter(t, np.float32(np.inf if k > 40 else -np.inf))
            cand[k, 0] = t
        ok = np.flatnonzero(cand[:, 0] / _radius(cand) == tau[v, 0])
        if ok.size:
            x[v] = cand[ok[np.argmin(np.abs(ok - 40))]]
    r = _radius(x)
    ok = (x[:, :PLANT] / r[:, None]) == tau
    hit = np.zeros(len(targets), bool)
    hit[slot[slot >= 0]] = ok[slot >= 0]
    return x, hit


def _codebook(kind, levels):
    if kind == "lloyd":
        return O.lloyd_max_codebook(D, {16: 4, 4: 2}[levels])[0].astype(np.float32)
    rng = np.random.default_rng(levels)
    if kind == "symmetric":          # c_i = -c_{L-1-i}, not Lloyd-Max: the probe near zero
        h = np.sort(rng.uniform(0.01, 0.45, levels // 2)).astype(np.float32)
        return np.concatenate([-h[::-1], h])
    if kind == "near_zero":          # a pair around zero, midpoint 2^-26: the 16-ary search
        h = np.sort(rng.uniform(0.01, 0.45, levels // 2)).astype(np.float32)
        cb = np.concatenate([-h[::-1], h])
        cb[levels // 2] = np.float32(h[0] + 2.0 ** -25)
        return cb
    if kind == "random":             # arbitrary switch points
        return np.sort(rng.uniform(-0.6, 0.6, levels)).astype(np.float32)
    if kind == "tiny_pair":          # switch point below 2^-60: the table is refused, the scan runs
        h = np.sort(rng.uniform(0.01, 0.45, levels // 2)).astype(np.float32)
        cb = np.concatenate([-h[::-1], h])
        cb[levels // 2 - 1], cb[levels // 2] = np.float32(-2.0 ** -70), np.float32(2.0 ** -70)
        return cb
    if kind == "crowded":            # two switch points in the cell around 51/512: refused
        c = np.float32(51 / 512)
        mid = [c - np.float32(2.0 ** -14), c, c + np.float32(2.0 ** -14)]
        lo = np.sort(rng.uniform(-0.6, 0.05, levels - 4))
        return np.concatenate([lo, mid, [0.3]]).astype(np.float32)
    raise ValueError(kind)


KINDS = ["lloyd", "symmetric", "near_zero", "random", "tiny_pair", "crowded"]


def _cell(t):
    """The table's cell of a direction: round-half-even of 512 t, + 513."""
    return int(np.rint(np.float64(t) * 512)) + 513


@pytest.mark.parametrize("levels", [16, 4])
@pytest.mark.parametrize("kind", KINDS)
def test_planted_directions_reach_their_targets(kind, levels):
    """The planting itself (CPU): nearly every target direction is hit
    exactly, every switch point among them, and each codebook takes the
    table-build route its name says."""
    cb = _codebook(kind, levels)
    assert (np.diff(cb) > 0).all()
    t = _targets(cb)
    x, hit = _plant(t, 7)
    assert hit.mean() > 0.995, hit.mean()
    assert np.array_equal(OC.c_rotate_fma(x, np.eye(D, dtype=np.float32)), x)
    keys = _switch_points(cb)
    sp = np.array([_kfloat(k) for k in keys], np.float32)
    assert np.isin(sp, t[hit]).all()
    z = levels // 2 - 1                                   # the pair around zero
    mid_key = _key(np.float32(0.5) * cb[z] + np.float32(0.5) * cb[z + 1])
    cells = [_cell(v) for v in sp]
    if kind in ("lloyd", "symmetric"):                    # midpoint 0, switch point off it
        assert mid_key == 0 and abs(keys[z]) > 8
    if kind == "near_zero":                               # neither probe: the 16-ary search
        assert mid_key != 0 and abs(keys[z] - mid_key) > 8
    if kind == "tiny_pair":
        assert abs(sp[z]) < 2.0 ** -60
    if kind == "crowded":
        assert len(set(cells)) < len(cells)
    if kind in ("lloyd", "symmetric", "near_zero", "random"):   # the table is built
        assert len(set(cells)) == len(cells) and (np.abs(sp) >= 2.0 ** -60).all() and (np.abs(sp) < 1).all()


@pytest.mark.gpu
@pytest.mark.parametrize("levels", [16, 4])
@pytest.mark.parametrize("kind", KINDS)
def test_table_matches_the_scan_at_switch_points_and_cell_boundaries(kind, levels):
    print(f"cells kind={kind} levels={levels}", flush=True)
    cb = _codebook(kind, levels)
    x, hit = _plant(_targets(cb), 7)
    n = x.shape[0]
    R = np.eye(D, dtype=np.float32)
    xt, Rt, cbt = (torch.from_numpy(a).to(DEV) for a in (x, R, cb))
    radius = torch.empty(n, device=DEV)
    packed = torch.empty(n, D // 2, dtype=torch.uint8, device=DEV)
    _lib.lib().polarquant_compress_cuda_c(xt.data_ptr(), Rt.data_ptr(), cbt.data_ptr(), radius.data_ptr(),
                                          packed.data_ptr(), n, D, levels, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    y = OC.c_rotate_fma(x, R)
    assert np.array_equal(y, x)           # R = I leaves each value as is (a zero may turn -0)
    r_ref, idx = OC.c_quantize_rotated(y, cb)
    assert np.array_equal(radius.cpu().numpy().view(np.uint32), r_ref.view(np.uint32))
    got = packed.cpu().numpy()
    got_idx = np.empty((n, D), np.int64)
    got_idx[:, 0::2], got_idx[:, 1::2] = got & 15, got >> 4
    bad = np.argwhere(got_idx != idx)
    assert bad.size == 0, [(int(v), int(j), float(x[v, j] / r_ref[v]), int(got_idx[v, j]), int(idx[v, j]))
                           for v, j in bad[:8]]


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [4, 2])
def test_block_encoder_table_at_switch_points_and_cell_boundaries(bits, monkeypatch):
    """The same planted directions through pqkv_encode's block output (fp32
    input: the register-blocked exact encoder) with the Lloyd-Max codebook."""
    print(f"cells block encoder bits={bits}", flush=True)
    monkeypatch.setenv("PQKV_ENCODE_KERNEL", "exact")
    cb = O.lloyd_max_codebook(D, bits)[0].astype(np.float32)
    x, _ = _plant(_targets(cb), 11)
    n = x.shape[0]
    R = np.eye(D, dtype=np.float32)
    cache = quantizer.allocate_cache(1, 1, n, D, bits, DEV)
    quantizer.compress_pq(torch.from_numpy(x).to(DEV).view(1, 1, n, D), torch.from_numpy(R).to(DEV), cache=cache)
    torch.cuda.synchronize()
    r_ref, idx = OC.c_quantize_rotated(OC.c_rotate_fma(x, R), cb)
    want = OC.c_pack_blocks(r_ref, idx, bits)
    got = cache.blocks.cpu().numpy().reshape(n, -1)
    assert np.array_equal(got, want), np.argwhere((got != want).any(axis=1))[:8].ravel().tolist()
