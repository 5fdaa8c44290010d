"""MI355X (gfx950) quantized-matmul backend for ggnpu.

The product is the C ABI in include/ggq.h, implemented by
ggnpu_amd/lib/libggq_hip.so (HIP kernels in ggnpu_amd/csrc).  This package
holds the ctypes binding (``ggnpu_amd.lib``), a Python mirror of ggnpu's
``Backend``/``MulMatParams`` interface (``ggnpu_amd.backend``), and the
in-tree build (``ggnpu_amd.build``).
"""
from .lib import load_library, GgqError, Status, GgmlType, ActMode  # noqa: F401
