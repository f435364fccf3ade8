"""src/polarquant_kv_cuda/inference/config.py:7-12."""

from polarquant_kv.inference import PolarQuantConfig  # noqa: F401
