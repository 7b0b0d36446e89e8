"""ctypes binding of libasdsl_hip.so (the C ABI declared in include/asdsl_hip.h).

The library is the only compute path: if it is missing this module raises at
import, and every call checks the returned status (argument errors become
``ValueError`` like the reference's ``std::invalid_argument``; HIP failures
become ``RuntimeError``).  There is no CPU fallback.

Buffers cross the boundary as raw device pointers.  ``torch`` is used only to
own device memory and to name the current stream.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

PKG_ROOT = Path(__file__).resolve().parent.parent
LIB_PATH = Path(os.environ.get("ASDSL_HIP_LIB", PKG_ROOT / "lib" / "libasdsl_hip.so"))

ASDSL_OK = 0
ASDSL_ERR_INVALID_ARGUMENT = 1
ASDSL_ERR_HIP = 2
ASDSL_ERR_UNSUPPORTED = 3

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float

# name -> argument types (return type is int status unless listed in _RESTYPE)
SIGNATURES: dict[str, list] = {
    "asdsl_abi_version": [],
    "asdsl_last_error": [],
    "asdsl_device_cu_count": [],
    "asdsl_reserve_workspace": [ctypes.c_size_t],
    "asdsl_profile_next_launch": [_P, _P],
    "asdsl_dequant_gguf_q4k": [_P, _P, _I, _I, _P],
    "asdsl_dequant_gguf_q6k": [_P, _P, _I, _I, _P],
    "asdsl_dequant_gguf_q5k": [_P, _P, _I, _I, _P],
    "asdsl_dequant_gguf_q8_0": [_P, _P, _I, _I, _P],
    "asdsl_dequant_gguf_q4_0": [_P, _P, _I, _I, _P],
    "asdsl_dequant_gguf_q4_1": [_P, _P, _I, _I, _P],
    "asdsl_dequant_gguf_q5_0": [_P, _P, _I, _I, _P],
    "asdsl_dequant_gguf_q5_1": [_P, _P, _I, _I, _P],
    "asdsl_dequant_gguf_q2k": [_P, _P, _I, _I, _P],
    "asdsl_dequant_gguf_q3k": [_P, _P, _I, _I, _P],
    "asdsl_repack_gguf_q4k_to_q4km": [_P, _P, _I, _I, _P],
    "asdsl_quantize_q4_symmetric": [_P, _P, _P, _P, _I, _I, _I, _P],
    "asdsl_profile_stages_begin": [_I],
    "asdsl_profile_stages_end": [_I, _P, _P, _P, _P],
    "asdsl_stream_read": [_P, ctypes.c_size_t, _P, _I, _P],
    "asdsl_stream_read_ex": [_P, ctypes.c_size_t, _P, _I, _I, _I, _I, _P],
    "asdsl_grid_sync_probe_work_bytes": [_I],
    "asdsl_grid_sync_probe": [_I, _I, _I, _P, ctypes.c_size_t, _I, _P],
    "asdsl_quantize_activation": [_P, _P, _P, _I, _I, _P],
    "asdsl_gemv_q4_32_preq": [_P, _P, _P, _P, _I, _I, _I, _P],
    "asdsl_gemv_q4_32_preq_fused": [_P, _P, _P, _I, _I, _I, _P],
    "asdsl_gemv_preq2_fused": [_P, _P, _P, _P, _I, _I, _I, _P],
    "asdsl_gemv_preq2_fused_batch": [_P, _P, _P, _P, _I, _I, _I, _I, _P],
    "asdsl_gemv_preq2": [_P, _P, _P, _P, _P, _I, _I, _I, _P],
    "asdsl_dequant_preq2": [_P, _P, _P, _I, _I, _I, _P],
    "asdsl_gemv_q4_128_preq": [_P, _P, _P, _P, _I, _I, _I, _P],
    "asdsl_gemv_q4_128_fused": [_P, _P, _P, _I, _I, _I, _P],
    "asdsl_gemv_q4_q8": [_P, _P, _P, _P, _I, _I, _I, _P],
    "asdsl_gemv_q4km_q8": [_P, _P, _P, _I, _I, _P],
    "asdsl_gemv_q4_s256": [_P, _P, _P, _P, _I, _I, _I, _P],
    "asdsl_gemv_q4_s256_fused": [_P, _P, _P, _I, _I, _P],
    "asdsl_gemv_q4_packed": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P],
    "asdsl_matmul_batch_q4": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P],
    "asdsl_gemm_q4_128": [_P, _P, _P, _I, _I, _I, _I, _P],
    "asdsl_gemv_q4_unpacked": [_P, _P, _P, _P, _P, _I, _I, _I, _P],
    "asdsl_gemv_q4_gs64": [_P, _P, _P, _P, _I, _I, _I, _P],
    "asdsl_gemv_q8_unpacked": [_P, _P, _P, _P, _P, _I, _I, _I, _P],
    "asdsl_compute_bitmask": [_P, _P, _I, _F, _P],
    "asdsl_gemv_sparse_unpacked": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _P],
    "asdsl_sparse_down_proj_T": [_P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _P],
    "asdsl_sparse_down_work_bytes": [_I],
    "asdsl_sparse_down_proj_T_noalloc": [_P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _P],
    "asdsl_sparse_down_proj_T_ws": [_P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _P, ctypes.c_size_t, _P],
    "asdsl_gemv_preq2_fused_batch_work_bytes": [_I],
    "asdsl_gemv_preq2_fused_batch_ws": [_P, _P, _P, _P, _I, _I, _I, _I, _P, ctypes.c_size_t, _P],
    "asdsl_affine_batch_work_bytes": [_I, _I, _I],
    "asdsl_gemv_q4_packed_ws": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P, ctypes.c_size_t, _P],
    "asdsl_gemv_q4_gs64_ws": [_P, _P, _P, _P, _I, _I, _I, _P, ctypes.c_size_t, _P],
    "asdsl_matmul_batch_q4_ws": [_P, _P, _P, _P, _P, _I, _I, _I, _I, _P, ctypes.c_size_t, _P],
    "asdsl_gemm_q4_128_ws": [_P, _P, _P, _I, _I, _I, _I, _P, ctypes.c_size_t, _P],
    "asdsl_gemv_sparse_with_indices": [_P, _P, _P, _P, _P, _I, _P, _I, _I, _I, _P, _P, _P],
    "asdsl_gemv_preq2_rmsnorm": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _P, _P],
    "asdsl_gemv_preq2_swiglu": [_P, _P, _P, _P, _I, _I, _I, _F, _P],
    "asdsl_gemv_preq2_rmsnorm_swiglu": [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _F, _F, _P],
    "asdsl_attention_work_floats": [_I, _I],
    "asdsl_attention_f16kv": [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P],
    "asdsl_attention_q8kv": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P],
    "asdsl_decode_work_bytes": [_P],
    "asdsl_decode_flags_offset": [_P],
    "asdsl_decode_token": [_P, _P, _P, _P, _P, _P],
    "asdsl_decode_token_upto": [_P, _P, _P, _I, _P, _P, _P],
    "asdsl_decode_verify_work_bytes": [_P, _I],
    "asdsl_decode_verify": [_P, _P, _I, _P, _P, _P, _P, _P],
    "asdsl_kv_zero_from": [_P, _P, _I, _I, _I, _I, _P],
    "asdsl_kv_zero_from_q8": [_P, _P, _P, _P, _I, _I, _I, _I, _P],
    "asdsl_repack_preq_to_preq2": [_P, _P, _P, _I, _I, _I, _P],
    "asdsl_repack_asym_to_q4_32": [_P, _P, _P, _P, _I, _I, _I, _P],
    "asdsl_repack_asym_to_preq2": [_P, _P, _P, _P, _P, _I, _I, _I, _P],
    "asdsl_repack_fp32_to_q4_128": [_P, _P, _I, _I, _I, _P],
    "asdsl_repack_asym_to_q4_128": [_P, _P, _P, _P, _I, _I, _I, _P],
    "asdsl_repack_q4_128_to_preq2": [_P, _P, _P, _I, _I, _P],
}
_RESTYPE = {"asdsl_last_error": ctypes.c_char_p, "asdsl_attention_work_floats": ctypes.c_size_t,
            "asdsl_decode_work_bytes": ctypes.c_size_t, "asdsl_decode_verify_work_bytes": ctypes.c_size_t,
            "asdsl_decode_flags_offset": ctypes.c_size_t,
            "asdsl_sparse_down_work_bytes": ctypes.c_size_t, "asdsl_grid_sync_probe_work_bytes": ctypes.c_size_t,
            "asdsl_gemv_preq2_fused_batch_work_bytes": ctypes.c_size_t,
            "asdsl_affine_batch_work_bytes": ctypes.c_size_t}


class HipLibraryMissing(ImportError):
    pass


def _load() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise HipLibraryMissing(
            f"{LIB_PATH} is not built; run `python asdsl-framework_amd/build_hip.py` "
            "(or __graft_entry__.build()). The HIP library is the only compute path."
        )
    # torch's HIP runtime must be the process's only one.  torch links its
    # bundled runtime by the name libamdhip64.so, this library by the soname
    # libamdhip64.so.7, which that runtime carries: loaded after torch, the
    # library binds to torch's runtime.  Loaded first, it pulls in the system
    # runtime and torch then loads its own beside it; with torch's initialised
    # first, this library's calls fail with hipErrorNoDevice.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name, None)
        if fn is None:
            continue  # reported by exported_symbols()/tests, not fatal for other entry points
        fn.argtypes = argtypes
        fn.restype = _RESTYPE.get(name, ctypes.c_int)
    return lib


LIB = _load()


def exported(name: str) -> bool:
    return getattr(LIB, name, None) is not None


def last_error() -> str:
    msg = LIB.asdsl_last_error()
    return msg.decode() if msg else ""


def check(status: int, fn: str) -> None:
    if status == ASDSL_OK:
        return
    msg = last_error() or f"{fn} failed with status {status}"
    if status == ASDSL_ERR_INVALID_ARGUMENT:
        raise ValueError(msg)
    raise RuntimeError(msg)


def call(name: str, *args) -> None:
    check(getattr(LIB, name)(*args), name)


# ----------------------------------------------------------------- buffers
def _torch():
    import torch  # imported lazily: argument checks must not need it

    return torch


def device() -> "torch.device":
    torch = _torch()
    if not torch.cuda.is_available():
        raise RuntimeError("no usable HIP device (torch.cuda.is_available() is False)")
    return torch.device("cuda", torch.cuda.current_device())


def stream_handle() -> int:
    torch = _torch()
    return int(torch.cuda.current_stream().cuda_stream)


_NP_TO_TORCH = {
    np.dtype(np.uint8): "uint8",
    np.dtype(np.int8): "int8",
    np.dtype(np.float32): "float32",
    np.dtype(np.int32): "int32",
    np.dtype(np.uint32): "int32",  # bit patterns; kernels read 32-bit words
}


def is_device_tensor(a) -> bool:
    torch = _torch()
    return isinstance(a, torch.Tensor) and a.is_cuda


def to_device(a, np_dtype) -> "torch.Tensor":
    """Device tensor with a's contents: zero-copy for a contiguous device tensor
    of the right dtype, otherwise a copy (numpy or host tensors are uploaded)."""
    torch = _torch()
    np_dtype = np.dtype(np_dtype)
    tdt = getattr(torch, _NP_TO_TORCH[np_dtype])
    if isinstance(a, torch.Tensor):
        t = a
        if t.dtype != tdt:
            if np_dtype == np.uint32 and t.dtype in (torch.int32,):
                pass
            else:
                t = t.to(tdt)
        if not t.is_cuda:
            t = t.to(device())
        return t.contiguous()
    arr = np.ascontiguousarray(a, dtype=np_dtype)
    if not arr.flags.writeable:  # a read-only memory map (a GGUF payload): torch needs writable memory
        arr = arr.copy()
    if np_dtype == np.uint32:
        arr = arr.view(np.int32)
    return torch.from_numpy(arr).to(device(), non_blocking=False)


def empty_device(shape, np_dtype) -> "torch.Tensor":
    torch = _torch()
    tdt = getattr(torch, _NP_TO_TORCH[np.dtype(np_dtype)])
    return torch.empty(shape, dtype=tdt, device=device())


def ptr(t) -> int:
    return int(t.data_ptr())


def cu_count() -> int:
    n = LIB.asdsl_device_cu_count()
    if n < 0:
        raise RuntimeError(last_error())
    return n


def profile_stages(run, max_launches: int = 4096) -> tuple[list[tuple[str, float]], float]:
    """Runs ``run()``, which queues this library's launches on the calling
    thread, with the stage recorder armed (asdsl_profile_stages_begin/_end):
    returns each launch's (stage label, ms) in launch order and the ms from the
    first launch's start to the last one's end.  Waits for the launches."""
    check(LIB.asdsl_profile_stages_begin(max_launches), "asdsl_profile_stages_begin")
    labels = (ctypes.c_char_p * max_launches)()
    ms = (ctypes.c_float * max_launches)()
    count, span = ctypes.c_int(0), ctypes.c_float(0.0)
    try:
        run()
    finally:
        status = LIB.asdsl_profile_stages_end(max_launches, labels, ms, ctypes.byref(count), ctypes.byref(span))
    check(status, "asdsl_profile_stages_end")
    return [(labels[i].decode(), float(ms[i])) for i in range(count.value)], float(span.value)
