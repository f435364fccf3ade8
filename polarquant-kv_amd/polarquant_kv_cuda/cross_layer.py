"""Cross-layer delta coding (src/polarquant_kv_cuda/cross_layer.py:19-102)."""

from polarquant_kv.policies import (differential_decode, differential_encode,  # noqa: F401
                                    estimate_differential_gain, measure_cross_layer_similarity)
