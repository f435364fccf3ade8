"""Write golden vectors for the parts of the path that no closed form pins.

Run in the build container only (the reference tree is not on the GPU box):

    python tests/golden/make_golden.py /root/reference

It imports three reference generators and records their outputs as fixtures:
  * build_lloyd_max_codebook  src/polarquant_kv_cuda/lloyd_max.py:12-79
    -> codebooks.json (centroids and boundaries, d in {64,128}, bits in {2,3,4})
  * generate_rotation_matrix  python/polarquant_kv/rotation.py:7-35
    -> R_d{64,128}_s42.npy (float64)
  * generate_jl_matrix        python/polarquant_kv/qjl.py:8-22
    -> P_m{m}_d{d}_s{seed}.npy (float64)
Only data is written; no reference source is copied.
"""

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))


def main(ref_root: str) -> None:
    sys.path.insert(0, os.path.join(ref_root, "src"))
    sys.path.insert(0, os.path.join(ref_root, "python"))
    from polarquant_kv_cuda.lloyd_max import build_lloyd_max_codebook
    from polarquant_kv.rotation import generate_rotation_matrix
    from polarquant_kv.qjl import generate_jl_matrix

    books = {}
    for d in (64, 128):
        for bits in (2, 3, 4):
            c, b = build_lloyd_max_codebook(d, bits)
            books[f"d{d}_b{bits}"] = {
                "centroids": [float(x) for x in np.asarray(c, np.float32)],
                "boundaries": [float(x) for x in np.asarray(b, np.float32)],
            }
    with open(os.path.join(HERE, "codebooks.json"), "w") as f:
        json.dump({"source": "src/polarquant_kv_cuda/lloyd_max.py:12-79 "
                             "(n_iterations=300, grid_size=50000)",
                   "codebooks": books}, f, indent=1)

    for d in (64, 128):
        np.save(os.path.join(HERE, f"R_d{d}_s42.npy"), generate_rotation_matrix(d, seed=42))
    for m, d, seed in ((64, 64, 43), (128, 128, 43), (64, 128, 42)):
        np.save(os.path.join(HERE, f"P_m{m}_d{d}_s{seed}.npy"), generate_jl_matrix(m, d, seed=seed))
    print("golden vectors written to", HERE)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
