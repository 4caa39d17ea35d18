"""exl3_amd: MI355X-native EXL3 trellis / GLM-5 MoE decode path.

The compute lives in libexl3moe.so (HIP, gfx950) behind the C ABI of
include/exl3_moe.h; this package is the host-side mirror of the reference's
trellis_gemm.h / glm5_moe.h call surface (trellis.py, moe.py), the build recipe
(build.py) and the seeded synthetic workloads (synth.py).
"""
from . import synth  # noqa: F401  (numpy only; importable without torch or a GPU)

__all__ = ["synth"]
