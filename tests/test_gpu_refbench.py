"""The reference benchmark's own flow (scripts/benchmark_turboquant.py:9-120)
through this build's import surface, at the published shapes: B = 1,
Hq = Hkv = 32, D = 128, S in {512, 2048, 4096} (README.md:120-122).

Imports as the script does (polarquant_kv_cuda.rotation / lloyd_max /
compress_kernel / compressor, polarquant_turboquant, polarquant_full), then:
- the "old C++" path: compress_gpu (group format) + full_compressed_attention,
  against the oracle's group attention on the decompressed caches;
- the TurboQuant path: turboquant_compress + turboquant_full_attention on the
  SoA cache, against the oracle's SoA attention on the same bytes;
- the script's accuracy and compression-ratio figures (cosine to SDPA on the
  fp16 K/V after the inverse rotation, 128 / 36 bytes)."""

import math

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("S", [512, 2048, 4096])
def test_reference_benchmark_flow(S):
    import polarquant_full
    import polarquant_turboquant
    from polarquant_kv_cuda.compress_kernel import compress_gpu
    from polarquant_kv_cuda.compressor import get_memory_bytes
    from polarquant_kv_cuda.lloyd_max import get_codebook_torch
    from polarquant_kv_cuda.rotation import generate_rotation_matrix

    print(f"reference benchmark flow S={S}", flush=True)
    D, Hq = 128, 32
    torch.manual_seed(42)
    R = generate_rotation_matrix(D, seed=42, device=DEV)
    k_cb = get_codebook_torch(D, 4, device=DEV)
    v_cb = get_codebook_torch(D, 4, device=DEV)
    Q = torch.randn(1, Hq, 1, D, dtype=torch.float16, device=DEV)
    K = torch.randn(1, Hq, S, D, dtype=torch.float16, device=DEV)
    V = torch.randn(1, Hq, S, D, dtype=torch.float16, device=DEV)
    scale = 1.0 / math.sqrt(D)
    Rn = R.double().cpu().numpy()

    # "Old C++": group format + polarquant_full
    ck = compress_gpu(K, R, n_bits=4, group_size=32)
    cv = compress_gpu(V, R, n_bits=4, group_size=32)
    assert get_memory_bytes(ck) > 0
    ng = D // 32
    q_f = Q.squeeze(2).float().reshape(Hq, D).contiguous()
    pk_old = ck.quantized_direction.reshape(Hq, S, -1).contiguous()
    km = ck.group_mins.float().reshape(Hq, S, ng).contiguous()
    ks = ck.group_scales.float().reshape(Hq, S, ng).contiguous()
    kr_old = ck.radius.float().reshape(Hq, S).contiguous()
    pv_old = cv.quantized_direction.reshape(Hq, S, -1).contiguous()
    vm = cv.group_mins.float().reshape(Hq, S, ng).contiguous()
    vs = cv.group_scales.float().reshape(Hq, S, ng).contiguous()
    vr_old = cv.radius.float().reshape(Hq, S).contiguous()
    out_old = torch.zeros(Hq, D, dtype=torch.float32, device=DEV)
    qr_old = torch.zeros(Hq, D, dtype=torch.float32, device=DEV)
    sc_old = torch.zeros(Hq, S, dtype=torch.float32, device=DEV)
    ao_old = torch.zeros(Hq, D, dtype=torch.float32, device=DEV)
    polarquant_full.full_compressed_attention(
        q_f.data_ptr(), R.data_ptr(), pk_old.data_ptr(), km.data_ptr(), ks.data_ptr(), kr_old.data_ptr(),
        pv_old.data_ptr(), vm.data_ptr(), vs.data_ptr(), vr_old.data_ptr(), out_old.data_ptr(), qr_old.data_ptr(),
        sc_old.data_ptr(), ao_old.data_ptr(), Hq, Hq, S, D, 32, ng, scale)
    torch.cuda.synchronize()
    # oracle: the group format's reconstruction in the rotated space, then
    # attention and the inverse rotation (float64)
    def rot_hat(c):
        return O.gpu_group_rotated(c.radius.float().cpu().numpy().reshape(-1),
                                   c.quantized_direction.cpu().numpy().reshape(Hq * S, -1),
                                   c.group_mins.float().cpu().numpy().reshape(Hq * S, ng),
                                   c.group_scales.float().cpu().numpy().reshape(Hq * S, ng), D, 4)
    Kh, Vh = rot_hat(ck).reshape(Hq, S, D), rot_hat(cv).reshape(Hq, S, D)
    q_rot64 = q_f.double().cpu().numpy() @ Rn.T
    want_old = np.stack([O.sdpa(q_rot64[h][None], Kh[h], Vh[h], scale)[0] for h in range(Hq)]) @ Rn
    assert np.abs(out_old.double().cpu().numpy() - want_old).max() <= 2e-3

    # TurboQuant path
    K_flat = K.reshape(-1, D).float().contiguous()
    V_flat = V.reshape(-1, D).float().contiguous()
    N = K_flat.shape[0]
    kr = torch.zeros(N, dtype=torch.float32, device=DEV)
    pk = torch.zeros(N, D // 2, dtype=torch.uint8, device=DEV)
    vr = torch.zeros(N, dtype=torch.float32, device=DEV)
    pv = torch.zeros(N, D // 2, dtype=torch.uint8, device=DEV)
    polarquant_turboquant.turboquant_compress(K_flat.data_ptr(), R.data_ptr(), k_cb.data_ptr(), kr.data_ptr(),
                                              pk.data_ptr(), N, D, 16)
    polarquant_turboquant.turboquant_compress(V_flat.data_ptr(), R.data_ptr(), v_cb.data_ptr(), vr.data_ptr(),
                                              pv.data_ptr(), N, D, 16)
    torch.cuda.synchronize()
    pk, kr, pv, vr = pk.reshape(Hq, S, -1), kr.reshape(Hq, S), pv.reshape(Hq, S, -1), vr.reshape(Hq, S)
    q_rot = (Q.squeeze(2).float() @ R.T).reshape(Hq, D).contiguous()
    out_tq = torch.zeros(Hq, D, dtype=torch.float32, device=DEV)
    sc_tq = torch.zeros(Hq, S, dtype=torch.float32, device=DEV)
    polarquant_turboquant.turboquant_full_attention(
        q_rot.data_ptr(), R.data_ptr(), pk.data_ptr(), kr.data_ptr(), pv.data_ptr(), vr.data_ptr(),
        k_cb.data_ptr(), v_cb.data_ptr(), out_tq.data_ptr(), q_rot.data_ptr(), sc_tq.data_ptr(),
        out_tq.data_ptr(), Hq, Hq, S, D, 16, scale)
    torch.cuda.synchronize()
    cb = O.lloyd_max_codebook(D, 4)[0]
    want_tq = O.decode_attention_soa(q_rot.cpu().numpy(), pk.reshape(Hq * S, -1).cpu().numpy(),
                                     kr.reshape(-1).cpu().numpy(), pv.reshape(Hq * S, -1).cpu().numpy(),
                                     vr.reshape(-1).cpu().numpy(), cb, Hq, scale)
    got = out_tq.double().cpu().numpy()
    assert np.abs(got - want_tq).max() <= 2e-3
    assert (got * want_tq).sum() / (np.linalg.norm(got) * np.linalg.norm(want_tq)) >= 0.9999

    # the script's accuracy and compression figures
    out_std = torch.nn.functional.scaled_dot_product_attention(Q.float(), K.float(), V.float()).half()
    out_final = (out_tq.reshape(1, Hq, D) @ R).half()
    cos = torch.nn.functional.cosine_similarity(out_std.flatten().float(), out_final.flatten().float(), dim=0)
    assert cos > 0.95, cos
    comp_ratio = (K.nelement() * 2 + V.nelement() * 2) / (pk.nelement() + kr.nelement() * 4 + pv.nelement() +
                                                          vr.nelement() * 4)
    assert abs(comp_ratio - 256 / 68) < 1e-9
