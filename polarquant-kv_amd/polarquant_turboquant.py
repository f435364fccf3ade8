"""Import name of the reference's pybind module (csrc/flash_turboquant.cu:227:
PYBIND11_MODULE(polarquant_turboquant, m)), so that callers written against it
(scripts/benchmark_turboquant.py) switch by putting this directory on the path.
The functions live in polarquant_kv.turboquant."""

from polarquant_kv.turboquant import turboquant_compress, turboquant_full_attention  # noqa: F401

__all__ = ["turboquant_compress", "turboquant_full_attention"]
