"""pb_amd — MI355X (gfx950) MoE block for pb's FlashMoE runtime.

The product is the C-ABI library ``libpbmoe.so`` (include/pbmoe.h) holding
hand-written HIP kernels; this package carries its sources (``csrc/``), the
build script, a ctypes binding (``abi``), the host-side mirror of the
reference operator seam (``flashmoe``), the seeded input generator
(``synth``) and the benchmark workload shapes C1-C5 (``configs``).
"""
from . import abi, configs, synth  # noqa: F401

__all__ = ["abi", "configs", "synth", "flashmoe"]
