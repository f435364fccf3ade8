"""Encoder parity over seeded random sizes: the vector count (tiny, one off
a 64-vector step, large), head_dim, width, data law, and the row split
(n_outer x n_inner). The matrix-core encoder's blocks and fp32 radii must
equal the C oracle's quantiser on the rotation it returns, bit for bit, as
in test_gpu_encode."""

import numpy as np
import pytest

import oracle as OC
from oracle import oracle as O
from polarquant_kv.lloyd_max import padded_codebook_torch
from test_gpu_encode import DEV, _encode_mfma, _fp16_inputs

pytestmark = pytest.mark.gpu


def _shape(seed):
    rng = np.random.default_rng(3000 + seed)
    n_inner = int(rng.choice([1, 2, 63, 64, 65, 127, 129, int(rng.integers(1, 5000))]))
    n_outer = int(rng.integers(1, 4))
    d = int(rng.choice([64, 128]))
    bits = int(rng.choice([2, 4]))
    kind = str(rng.choice(["normal", "channel", "special"]))
    return n_outer, n_inner, d, bits, kind


@pytest.mark.parametrize("seed", range(16))
def test_encode_mfma_random_sizes(seed):
    n_outer, n_inner, d, bits, kind = _shape(seed)
    n = n_outer * n_inner
    if kind == "special" and n < 5:
        kind = "normal"                                    # the special rows need five vectors
    print(f"encode sweep seed {seed}: n={n_outer}x{n_inner} d={d} bits={bits} {kind}", flush=True)
    x = _fp16_inputs(n, d, seed, kind)
    R32 = O.rotation_matrix(d, 42).astype(np.float32)
    blocks, rot = _encode_mfma(x, R32, padded_codebook_torch(d, bits, DEV), bits, d, n_outer=n_outer)
    r_ref, idx_ref = OC.c_quantize_rotated(rot, O.lloyd_max_codebook(d, bits)[0])
    assert np.array_equal(blocks, OC.c_pack_blocks(r_ref, idx_ref, bits))
    assert np.array_equal(_encode_mfma.radius.view(np.uint32), r_ref.view(np.uint32))
