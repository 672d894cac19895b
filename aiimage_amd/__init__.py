"""aiimage_amd: MI355X-native quantized decode-linear path of Aexis (newzjh/AIImage).

The compute lives in libaexq.so (hand-written HIP for gfx950, C ABI in
include/aexq.h).  This package holds its build step (aiimage_amd.build), the
ctypes binding (aiimage_amd._abi) and the host-side mirror of the reference's
Gemm operator (aiimage_amd.aexq).  Importing aiimage_amd.aexq requires the
built library; there is no CPU fallback.
"""

__all__ = ["build", "aexq", "synth"]
