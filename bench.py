#!/usr/bin/env python3
"""PQ4 decode-attention throughput on one MI355X (plus encode tokens/s).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

Workload (the 32K-context metric config): one
Llama-3-8B-shaped attention layer, B=8, 32 query / 8 kv heads, d=128, 32768
cached tokens. K and V are synthetic fp16 with per-(head, channel) std drawn
from LogNormal(0, 1) and 1 % of the channels scaled x20, seeded. The whole
cache (K and V) is PQ4-encoded on the GPU, then a "step" is one decode
attention call for the batch (query rotation, split-K attention over the
compressed cache, merge + inverse rotation). Inputs are resident in HBM before
the timed region.

value = algorithmic bytes per step (compressed K+V read once, query read,
output written) / step time. roofline: the split-K decode kernel's algorithmic
bytes per launch over its mean duration, timed with hipEvents that the library
records on the launch stream in a second loop of `--steps` calls (the timed
loop runs without them); roofline.traffic is the HBM bytes per launch of
that kernel from the committed rocprofv3 counter summary
(profiles/decode_mfma_config3_hbm_traffic.md: FETCH_SIZE and WRITE_SIZE, each
scaled by the same counter's reading on a plain 1 GiB device copy, which
`--calibrate` adds after the timed region). cpu_baseline: the CPU oracle
(float64 numpy decode, one thread) over whole (batch, kv-head) streams of the
same cache for about 8 s, and the C oracle's encoder for about 4 s.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(ROOT, "polarquant-kv_amd"), ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_mfma_config3_hbm_traffic.md")
METRIC = "PQ4 decode-attn GB/s & % HBM peak; encode tokens/s; at 1 MI355X, 32K ctx"


def synth_channel_kv(torch, B, H, S, d, seed, dev):
    """fp16 [B, H, S, d]: N(0,1) times a per-(head, channel) LogNormal(0,1)
    std, with 1 % of the channels (at least one) of each head scaled x20."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    std = torch.exp(torch.randn(1, H, 1, d, generator=g, device=dev))
    n_out = max(1, round(0.01 * d))
    for h in range(H):
        ch = torch.randperm(d, generator=g, device=dev)[:n_out]
        std[0, h, 0, ch] *= 20.0
    x = torch.randn(B, H, S, d, generator=g, device=dev, dtype=torch.float32)
    return (x * std).clamp_(-65504, 65504).to(torch.float16)


def cpu_baseline(kc, vc, q, R, d, budget_s=8.0):
    """Time the CPU oracle's decode (float64 numpy, one thread) over whole
    (batch, kv-head) streams of the same cache until `budget_s` has elapsed.
    Returns (GB/s of compressed cache + query/output bytes, streams, seconds)."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle import oracle as O

    B, Hkv = kc.batch, kc.num_heads
    G = q.shape[1] // Hkv
    kb_all = kc.blocks.cpu().numpy()
    vb_all = vc.blocks.cpu().numpy()
    q_all = q.float().cpu().numpy().astype(np.float64)
    cb = O.lloyd_max_codebook(d, 4)[0]
    Rn = R.cpu().numpy().astype(np.float64)
    done_bytes, streams, elapsed = 0, 0, 0.0
    with threadpool_limits(limits=1):
        O.decode_attention(q_all[:1, :G], kb_all[:1, :1, :256], vb_all[:1, :1, :256], Rn, cb, cb)  # warm-up
        while elapsed < budget_s and streams < B * Hkv * 8:
            b, h = divmod(streams % (B * Hkv), Hkv)
            kb, vb = kb_all[b:b + 1, h:h + 1], vb_all[b:b + 1, h:h + 1]
            qs = q_all[b:b + 1, G * h:G * (h + 1)]
            t0 = time.perf_counter()
            O.decode_attention(qs, kb, vb, Rn, cb, cb)
            elapsed += time.perf_counter() - t0
            done_bytes += kb.nbytes + vb.nbytes + qs.size * 2 * 2
            streams += 1
    return done_bytes / elapsed / 1e9, streams, elapsed


def cpu_encode_baseline(d, budget_s=4.0, n=4096):
    """C oracle (single thread): FMA-chain rotation + quantiser + packing of
    n-vector batches until `budget_s` has elapsed. Returns vectors/s."""
    import numpy as np

    import oracle as OC
    from oracle import oracle as O

    x = np.random.default_rng(0).standard_normal((n, d)).astype(np.float32)
    R = O.rotation_matrix(d, 42).astype(np.float32)
    cb = O.lloyd_max_codebook(d, 4)[0]
    OC.c_rotate_fma(x[:64], R)
    vectors, elapsed = 0, 0.0
    while elapsed < budget_s:
        t0 = time.perf_counter()
        y = OC.c_rotate_fma(x, R)
        r, idx = OC.c_quantize_rotated(y, cb)
        OC.c_pack_blocks(r, idx, 4)
        elapsed += time.perf_counter() - t0
        vectors += n
    return vectors / elapsed


def decode_kernel_name(d: int) -> str:
    """The split kernel pqkv_decode_attn launches for a uniform PQ4 cache."""
    if os.environ.get("PQKV_DECODE_KERNEL", "") == "valu":
        return f"decode_split_kernel<{d},4,4,4>"
    return f"decode_mfma_kernel<{d},4,4,4>"


def committed_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed counter summary, or
    None when the summary is absent or covers another kernel."""
    try:
        with open(TRAFFIC_FILE) as f:
            fields = dict(line.split("=", 1) for line in f.read().splitlines() if line.startswith("- ") and "=" in line)
    except OSError:
        return None
    fields = {k[2:].strip(): v.strip().strip("`") for k, v in fields.items()}
    if fields.get("kernel") != kernel:
        return None
    return int(float(fields["traffic_bytes_per_launch"]))


def calibrate(torch, dev):
    """Untimed: a plain 1 GiB device-to-device copy (the runtime's copy
    kernel, 16-byte loads and stores like the decode kernel) whose FETCH_SIZE
    and WRITE_SIZE readings scale those counters to bytes."""
    x = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    y = torch.empty_like(x)
    x.fill_(1)
    y.copy_(x)
    torch.cuda.synchronize()
    del x, y


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--workload", choices=("config3", "config4", "config5"), default="config3",
                    help="config3 (default): the metric line; config4 / config5: the low-bit + QJL decode and "
                         "the chunked-prefill configurations, for their own measurement lines")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--encode-iters", type=int, default=3)
    ap.add_argument("--calibrate", action="store_true",
                    help="after the timed region, run a plain 1 GiB device copy (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the path shards by (batch, kv-head) with no exchange); "
              f"--gpus {args.gpus} is not supported", file=sys.stderr)
        return 2

    if args.workload == "config4":
        return run_config4(args)
    if args.workload == "config5":
        return run_config5(args)
    return run_config3(args)


def run_config3(args) -> int:
    import torch

    from polarquant_kv import _lib, attention, quantizer

    dev = "cuda:0"
    B, Hq, Hkv, S, d = 8, 32, 8, 32768, 128
    from oracle import oracle as O
    R = torch.from_numpy(O.rotation_matrix(d, 42).astype("float32")).to(dev)
    K = synth_channel_kv(torch, B, Hkv, S, d, 1234, dev)
    V = synth_channel_kv(torch, B, Hkv, S, d, 5678, dev)
    kc = quantizer.allocate_cache(B, Hkv, S, d, 4, dev)
    vc = quantizer.allocate_cache(B, Hkv, S, d, 4, dev)

    # ---- encode (full cache, K and V) ----
    _lib.profile_enable(True)
    quantizer.compress_pq(K, R, cache=kc, start=0)
    quantizer.compress_pq(V, R, cache=vc, start=0)
    torch.cuda.synchronize()
    _lib.profile_collect("encode")
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.encode_iters):
        quantizer.compress_pq(K, R, cache=kc, start=0)
        quantizer.compress_pq(V, R, cache=vc, start=0)
    e1.record()
    torch.cuda.synchronize()
    enc_ms = e0.elapsed_time(e1) / args.encode_iters
    enc_kernel_ms, enc_launches = _lib.profile_collect("encode")
    enc_tokens_s = B * S / (enc_ms / 1e3)
    enc_bytes = 2 * (K.numel() * 2 + kc.blocks.numel())
    del K, V

    # ---- decode ----
    # Timed region: library event hooks off (each hook pair costs ~6 us of
    # stream time). A second loop of the same length then records the hooks'
    # hipEvents on the launch stream for the per-kernel means.
    _lib.profile_enable(False)
    q = torch.randn(B, Hq, d, device=dev, dtype=torch.float16)
    ws = torch.empty(_lib.lib().pqkv_decode_workspace_bytes(B, Hq, Hkv, S, d), dtype=torch.uint8, device=dev)
    for _ in range(args.warmup):
        attention.decode_attention(q, kc, vc, R, workspace=ws)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(args.steps):
        out = attention.decode_attention(q, kc, vc, R, workspace=ws)
    t1.record()
    torch.cuda.synchronize()
    step_ms = t0.elapsed_time(t1) / args.steps
    _lib.profile_enable(True)
    _lib.profile_collect("")
    for _ in range(args.steps):
        attention.decode_attention(q, kc, vc, R, workspace=ws)
    torch.cuda.synchronize()
    split_ms, split_n = _lib.profile_collect("decode_split")
    merge_ms, merge_n = _lib.profile_collect("decode_merge")
    rot_ms, rot_n = _lib.profile_collect("decode_rotate")
    _lib.profile_enable(False)
    assert torch.isfinite(out.float()).all()

    cache_bytes = kc.blocks.numel() + vc.blocks.numel()            # 301 989 888
    qo_bytes = B * Hq * d * 2 * 2                                  # fp16 query in, fp16 output out
    step_bytes = cache_bytes + qo_bytes
    value = step_bytes / (step_ms / 1e3) / 1e9
    kern_ms = split_ms / max(split_n, 1)
    kern_bytes = cache_bytes + B * Hq * d * 4                      # compressed K+V + fp32 rotated query
    achieved = kern_bytes / (kern_ms / 1e3) / 1e9

    if args.calibrate:
        calibrate(torch, dev)

    kernel = decode_kernel_name(d)
    traffic = committed_traffic(kernel)
    cpu = None
    if not args.no_cpu:
        gbs, streams, t = cpu_baseline(kc, vc, q, R, d)
        enc_vs = cpu_encode_baseline(d)
        cpu = {"value": round(gbs, 4), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"oracle float64 numpy decode, one thread, of {streams} whole (batch, kv-head) streams "
                         f"of the same cache (S=32768, {Hq // Hkv} query heads each; 64 streams = one step) "
                         f"in {t:.1f} s; encode: C oracle FMA rotation + quantiser + packing, one thread, "
                         f"{enc_vs:.0f} vectors/s = {enc_vs / (2 * Hkv):.0f} tokens/s (K+V of {Hkv} kv heads)"}

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(step_ms, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "u4 codes; f16 hi/lo MFMA, f32 accumulate", "data": "synthetic",
        "config": {"workload": "config3: Llama-3-8B layer decode, B=8 Hq=32 Hkv=8 d=128 S=32768, PQ4 K+V "
                               "(block_pq4 72 B/vector), per-channel LogNormal(0,1) std + 1% x20 outliers",
                   "global_batch": B, "seq_len": S, "parallelism": "single GPU"},
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": kernel, "kernel_ms": round(kern_ms, 5),
                     "bytes_per_launch": kern_bytes},
        "stages_ms": {"query_rotate": round(rot_ms / max(rot_n, 1), 5), "split": round(kern_ms, 5),
                      "merge": round(merge_ms / max(merge_n, 1), 5)},
        "encode": {"tokens_per_s": round(enc_tokens_s), "ms": round(enc_ms, 4),
                   "kernel_ms": round(enc_kernel_ms / max(enc_launches, 1), 4), "GB_per_s": round(
                       enc_bytes / (enc_ms / 1e3) / 1e9, 2), "vectors": 2 * B * Hkv * S,
                   "kernel": "encode_mfma_kernel (matrix-core rotation, bit-exact quantiser)",
                   "roofline": {"bound": "hbm", "bytes": enc_bytes, "achieved_GBps": round(
                       enc_bytes / (enc_kernel_ms / max(enc_launches, 1) * 2 / 1e3) / 1e9, 2),
                       "frac": round(enc_bytes / (enc_kernel_ms / max(enc_launches, 1) * 2 / 1e3) / 1e9
                                     / HBM_PEAK_GBS, 4)}},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))
    return 0


def _timed(torch, fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        out = fn()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps, out


def _kernel_means(torch, _lib, fn, steps, names):
    """Kernel time per step (all launches of a kernel in one step summed),
    from the library's hipEvents on the launch stream."""
    _lib.profile_enable(True)
    _lib.profile_collect("")
    for _ in range(steps):
        fn()
    torch.cuda.synchronize()
    res = {}
    for n in names:
        ms, _ = _lib.profile_collect(n)
        res[n] = ms / steps
    _lib.profile_enable(False)
    return res


def run_config4(args) -> int:
    """Low-bit decode: B=4, 32 q / 8 kv heads, d=128, S=16384, keys with the
    QJL sign sketch (m = d, P seed 43); (i) 2-bit K and V, (ii) kv heads 0-3
    at 4 bits and 4-7 at 2 bits. value = variant (i)'s algorithmic GB/s."""
    import numpy as np
    import torch

    from oracle import oracle as O
    from polarquant_kv import _lib, attention, quantizer

    dev = "cuda:0"
    B, Hq, Hkv, S, d = 4, 32, 8, 16384, 128
    R64 = O.rotation_matrix(d, 42)
    R = torch.from_numpy(R64.astype("float32")).to(dev)
    P_rot = torch.from_numpy((O.jl_matrix(d, d, 43) @ R64.T).astype("float32")).to(dev)
    K = synth_channel_kv(torch, B, Hkv, S, d, 4321, dev)
    V = synth_channel_kv(torch, B, Hkv, S, d, 8765, dev)
    q = torch.randn(B, Hq, d, device=dev, dtype=torch.float16)
    variants = {"2bit": 2, "mixed": (4, 4, 4, 4, 2, 2, 2, 2)}
    res = {}
    for name, bits in variants.items():
        kc = quantizer.allocate_cache(B, Hkv, S, d, bits, dev, jl_dim=d)
        vc = quantizer.allocate_cache(B, Hkv, S, d, bits, dev)
        quantizer.compress_pq(K, R, cache=kc, jl_rot=P_rot)
        quantizer.compress_pq(V, R, cache=vc)
        ws = torch.empty(_lib.lib().pqkv_decode_workspace_bytes(B, Hq, Hkv, S, d), dtype=torch.uint8, device=dev)

        def step():
            return attention.decode_attention(q, kc, vc, R, jl_rot=P_rot, workspace=ws)

        _lib.profile_enable(False)
        step_ms, out = _timed(torch, step, args.steps, args.warmup)
        assert torch.isfinite(out.float()).all()
        km = _kernel_means(torch, _lib, step, args.steps, ("decode_split", "decode_merge", "decode_rotate"))
        cache_bytes = kc.blocks.numel() + vc.blocks.numel() + kc.qjl_signs.numel()
        step_bytes = cache_bytes + B * Hq * d * 2 * 2
        kern_bytes = cache_bytes + B * Hq * d * 4 + d * d * 4
        res[name] = {"ms_per_step": round(step_ms, 5), "GB_per_s": round(step_bytes / (step_ms / 1e3) / 1e9, 2),
                     "bytes_per_step": step_bytes, "split_ms": round(km["decode_split"], 5),
                     "split_GB_per_s": round(kern_bytes / (km["decode_split"] / 1e3) / 1e9, 2),
                     "merge_ms": round(km["decode_merge"], 5), "rotate_ms": round(km["decode_rotate"], 5)}
        del kc, vc
    v = res["2bit"]
    line = {
        "metric": "decode-attn GB/s at 1 MI355X (low-bit + QJL)", "value": v["GB_per_s"], "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": v["ms_per_step"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u2/u4 codes + 1-bit QJL signs; f16 hi/lo MFMA, f32 accumulate", "data": "synthetic",
        "config": {"workload": "config4: Llama-3-8B layer decode, B=4 Hq=32 Hkv=8 d=128 S=16384, QJL keys m=128 "
                               "(P seed 43); variants 2bit (block_pq2 K+V) and mixed (kv heads 0-3 PQ4, 4-7 PQ2)",
                   "global_batch": B, "seq_len": S, "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": v["split_GB_per_s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(v["split_GB_per_s"] / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "decode_mfma_kernel<128,4,2,2,qjl>", "kernel_ms": v["split_ms"]},
        "variants": res, "cpu_baseline": None,
    }
    print(json.dumps(line))
    return 0


def run_config5(args) -> int:
    """Chunked prefill: B=1, 64 q / 8 kv heads, d=128, 131072 cached PQ4
    tokens + a 2048-token fp16 chunk, causal. A step encodes the chunk's K
    and V into the cache and runs prefill attention for the chunk. value =
    algorithmic TFLOP/s of the attention (64 (2048 131072 + 2048 2049 / 2) 4 128)."""
    import torch

    from oracle import oracle as O
    from polarquant_kv import _lib, attention, quantizer

    dev = "cuda:0"
    B, Hq, Hkv, d = 1, 64, 8, 128
    S_cache, Sq = 131072, 2048
    S = S_cache + Sq
    R = torch.from_numpy(O.rotation_matrix(d, 42).astype("float32")).to(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    kc = quantizer.allocate_cache(B, Hkv, S, d, 4, dev)
    vc = quantizer.allocate_cache(B, Hkv, S, d, 4, dev)
    quantizer.compress_pq(torch.randn(B, Hkv, S_cache, d, generator=g, device=dev).half(), R, cache=kc)
    quantizer.compress_pq(torch.randn(B, Hkv, S_cache, d, generator=g, device=dev).half(), R, cache=vc)
    k_new = torch.randn(B, Hkv, Sq, d, generator=g, device=dev).half()
    v_new = torch.randn(B, Hkv, Sq, d, generator=g, device=dev).half()
    q = torch.randn(B, Hq, Sq, d, generator=g, device=dev).half()

    def step():
        quantizer.compress_pq(k_new, R, cache=kc, start=S_cache)
        quantizer.compress_pq(v_new, R, cache=vc, start=S_cache)
        return attention.prefill_attention(q, kc, vc, R, q_start=S_cache, causal=True)

    steps = max(1, min(args.steps, 20))
    _lib.profile_enable(False)
    step_ms, out = _timed(torch, step, steps, max(1, min(args.warmup, 3)))
    assert torch.isfinite(out.float()).all()
    km = _kernel_means(torch, _lib, step, steps, ("prefill_attn", "prefill_rotate", "prefill_out_rotate", "encode"))
    flops = 64 * (Sq * S_cache + Sq * (Sq + 1) / 2) * 4 * d
    tflops = flops / (step_ms / 1e3) / 1e12
    kern_tflops = flops / (km["prefill_attn"] / 1e3) / 1e12
    line = {
        "metric": "chunked-prefill attention TFLOP/s at 1 MI355X", "value": round(tflops, 2), "unit": "TFLOP/s",
        "n_gpus": 1, "steps": steps, "warmup": max(1, min(args.warmup, 3)), "ms_per_step": round(step_ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u4 codes; f16 hi/lo MFMA (3 products), f32 accumulate", "data": "synthetic",
        "config": {"workload": "config5: 70B-shaped layer prefill, B=1 Hq=64 Hkv=8 d=128, 131072 cached PQ4 "
                               "tokens + 2048-token fp16 chunk (encoded into the cache each step), causal; "
                               "K/V/Q N(0,1)",
                   "global_batch": B, "seq_len": S, "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(kern_tflops, 2), "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(kern_tflops / 2500.0, 4), "traffic": None, "kernel": "prefill_mfma_kernel<128>",
                     "kernel_ms": round(km["prefill_attn"], 4), "flops_per_launch": flops,
                     "note": "fp32-grade products cost 3 fp16 MFMAs each: this arithmetic tops out at 1/3"},
        "stages_ms": {k: round(v, 4) for k, v in km.items()},
        "cpu_baseline": None,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
