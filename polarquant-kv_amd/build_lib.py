"""Build libpqkv_hip.so for gfx950 with hipcc (no cmake, no torch extension).

    python polarquant-kv_amd/build_lib.py [--jobs N]

Each translation unit is compiled to an object in _build/ (git-ignored), then
linked in-tree as polarquant-kv_amd/polarquant_kv/_lib/libpqkv_hip.so, which
travels with the source tree to the GPU box.
"""

from __future__ import annotations

import argparse
import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "polarquant_kv", "_lib")
LIB = os.path.join(OUT_DIR, "libpqkv_hip.so")
BUILD = os.path.join(HERE, "_build")
SOURCES = ["pqkv_encode.hip", "pqkv_encode_tiled.hip", "pqkv_encode_mfma.hip", "pqkv_decode.hip", "pqkv_decode_mfma.hip",
           "pqkv_decode_mfma_k4v4_shared.hip", "pqkv_decode_mfma_k4v4_own.hip", "pqkv_decode_mfma_k4v2.hip",
           "pqkv_decode_mfma_k2v4.hip", "pqkv_decode_mfma_k2v2.hip", "pqkv_decode_mfma_pair.hip",
           "pqkv_decode_mfma_soa.hip", "pqkv_decode_mfma_paged_k4v4_shared.hip", "pqkv_decode_mfma_paged_k4v4_own.hip",
           "pqkv_decode_mfma_paged_k2v2.hip", "pqkv_decode_mfma_ggml.hip", "pqkv_prefill.hip", "pqkv_group.hip", "pqkv_group_gpu.hip", "pqkv_group_api.cpp",
           "pqkv_api.cpp", "pqkv_compat.cpp", "pqkv_ggml.cpp", "pqkv_noalloc.hip"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


COMMON = ["-O3", "-fPIC", "-std=c++17", "--offload-arch=gfx950", "-Wall", "-Wno-unused-function",
          # packed fp32 arithmetic stays disabled in device code
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


# Per-unit device flags. The 4-bit-key split-decode units schedule for
# instruction-level parallelism: their loop is latency-bound at two waves per
# SIMD, and the ILP scheduler keeps them within 256 VGPRs without spills
# (config-3 split kernel 0.4-0.9 us faster, config 2 0.2 us). The 2-bit-key
# units ran 0.4 us slower under it, the ggml and SoA units spill, and the
# encode and prefill kernels run slower, so they keep the default scheduler.
ILP = ["-mllvm", "-amdgpu-sched-strategy=max-ilp"]
UNIT_FLAGS = {f: ILP for f in ("pqkv_decode_mfma_k4v4_shared.hip", "pqkv_decode_mfma_k4v4_own.hip",
                               "pqkv_decode_mfma_k4v2.hip", "pqkv_decode_mfma_paged_k4v4_shared.hip",
                               "pqkv_decode_mfma_paged_k4v4_own.hip")}


def _headers_mtime() -> float:
    hs = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")]
    hs.append(os.path.join(HERE, "..", "include", "pqkv.h"))
    return max(os.path.getmtime(h) for h in hs if os.path.exists(h))


def compile_one(src: str, changed_only: bool = False) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    path = os.path.join(CSRC, src)
    if changed_only and os.path.exists(obj) and \
            os.path.getmtime(obj) > max(os.path.getmtime(path), _headers_mtime()):
        return obj
    if src.endswith(".hip"):
        cmd = [hipcc(), *COMMON, *UNIT_FLAGS.get(src, []), "-x", "hip", "-c", path, "-o", obj]
    else:
        # host-only units (validation, C ABI, the ggml type's CPU traits): plain
        # g++ against the HIP headers; no contraction, so host arithmetic
        # rounds where the source says
        cmd = ["g++", "-O2", "-fPIC", "-std=c++17", "-Wall", "-ffp-contract=off", "-D__HIP_PLATFORM_AMD__",
               "-I/opt/rocm/include", "-c", path, "-o", obj]
    subprocess.run(cmd, check=True)
    return obj


def build(jobs: int = 8, changed_only: bool = False) -> str:
    """Compile every unit (changed_only: only those older than their source
    or any header) and link the library."""
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(OUT_DIR, exist_ok=True)
    # the slowest units first, so that they overlap the rest
    order = sorted(SOURCES, key=lambda f: -os.path.getsize(os.path.join(CSRC, f)))
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(lambda f: compile_one(f, changed_only), order))
    tmp = LIB + ".tmp"
    subprocess.run([hipcc(), "-shared", "-fPIC", "--offload-arch=gfx950", *objs, "-o", tmp], check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=8)
    ap.add_argument("--changed", action="store_true", help="recompile only units older than their sources")
    args = ap.parse_args()
    print(build(args.jobs, args.changed))
