"""ditserve_amd — MI355X-native per-step DiT forward for ditserve (Wan2.1/Wan2.2, SD3.5).

All compute runs in hand-written gfx950 HIP kernels exported by libditk.so
(C ABI, see include/ditk.h).  Importing this package never touches the GPU;
ops raise if the library is not built.
"""
__version__ = "0.1.0"

from . import ops  # noqa: F401
