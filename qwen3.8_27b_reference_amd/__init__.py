"""MI355X (gfx950) GGUF Q4_K / Q6_K matmul with the block dequant fused into CDNA4 MFMA.

The product is libqk.so (HIP kernels + the C ABI declared in include/qk.h), built in-tree by
build.py.  This package holds its ctypes binding (qk.py) and a small ctypes HIP runtime wrapper
(hiprt.py) used for device buffers and streams.  Loading the binding fails loudly when libqk.so
has not been built: there is no CPU fallback.
"""
from . import hiprt, qk
from .qk import LAYOUT_GGUF, LAYOUT_T16, T_Q4_K, T_Q6_K, Lib, QkError, Weight

__all__ = ["hiprt", "qk", "Lib", "QkError", "Weight", "T_Q4_K", "T_Q6_K", "LAYOUT_GGUF", "LAYOUT_T16"]
