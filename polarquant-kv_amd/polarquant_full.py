"""Import name of the reference's pybind module polarquant_full
(csrc/polarquant_full.cu:184: PYBIND11_MODULE(polarquant_full, m)), called by
scripts/benchmark_turboquant.py:63-69. The function lives in
polarquant_kv.turboquant."""

from polarquant_kv.turboquant import full_compressed_attention  # noqa: F401

__all__ = ["full_compressed_attention"]
