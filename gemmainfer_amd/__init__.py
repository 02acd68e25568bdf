"""MI355X (gfx950) Token-Union W4A16 MoE path for GemmaInfer.

Hand-written HIP kernels behind a C ABI (``include/gemmainfer_amd.h``,
``gemmainfer_amd/lib/libgemmainfer_amd.so``), bound with ctypes.  The
``gemmainfer_csrc`` package at the repository root is the drop-in module the
reference engine imports; ``gemmainfer_amd.ops`` holds the torch-facing
wrappers it uses for device tensors.
"""
from . import ops  # noqa: F401
from ._lib import GIError, LIB_PATH  # noqa: F401

__all__ = ["ops", "GIError", "LIB_PATH"]
