"""HIP (gfx950) implementations of the reference's GEMV kernel API.

Mirrors asdsl/kernels/__init__.py of the reference: the pybind-module
stand-ins (``_native_gemv`` ...) keep the reference's function names and
arguments; every call runs on the GPU through libasdsl_hip.so.
"""

from asdsl.kernels import _native_gemv  # noqa: F401
