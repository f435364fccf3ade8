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
SOURCES = ["pqkv_encode.hip", "pqkv_encode_mfma.hip", "pqkv_decode.hip", "pqkv_decode_mfma.hip", "pqkv_prefill.hip",
           "pqkv_api.cpp", "pqkv_compat.cpp", "pqkv_noalloc.hip"]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


COMMON = ["-O3", "-fPIC", "-std=c++17", "--offload-arch=gfx950", "-Wall", "-Wno-unused-function",
          # packed fp32 arithmetic stays disabled in device code
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def compile_one(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    path = os.path.join(CSRC, src)
    if src.endswith(".hip"):
        cmd = [hipcc(), *COMMON, "-x", "hip", "-c", path, "-o", obj]
    else:
        # host-only units (validation, C ABI): plain g++ against the HIP headers
        cmd = ["g++", "-O2", "-fPIC", "-std=c++17", "-Wall", "-D__HIP_PLATFORM_AMD__",
               "-I/opt/rocm/include", "-c", path, "-o", obj]
    subprocess.run(cmd, check=True)
    return obj


def build(jobs: int = 4) -> str:
    os.makedirs(BUILD, exist_ok=True)
    os.makedirs(OUT_DIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    tmp = LIB + ".tmp"
    subprocess.run([hipcc(), "-shared", "-fPIC", "--offload-arch=gfx950", *objs, "-o", tmp], check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    print(build(ap.parse_args().jobs))
