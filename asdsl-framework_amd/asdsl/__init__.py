"""MI355X-native (gfx950 HIP) drop-in for the ASDSL batch-1 decode GEMV path.

``asdsl.kernels`` mirrors the reference's Python kernel API and its pybind11
modules (``_native_gemv``, ``_native_gemv_q8``, ``_native_sparse_gemv``); all
compute runs in ``lib/libasdsl_hip.so`` through the C ABI of include/asdsl_hip.h.
``asdsl.quantization`` produces the byte layouts those kernels read.
"""

__version__ = "0.1.0"
