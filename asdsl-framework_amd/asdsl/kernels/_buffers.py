"""Argument marshalling for one C-ABI call.

Inputs accept numpy arrays, host tensors or device tensors and are forced to
the kernel's dtype (the reference's pybind ``forcecast``).  Outputs are either
device tensors (written in place, asynchronously) or numpy arrays (a device
temporary is written and copied back after the call, which synchronizes the
stream).  Every buffer is checked to hold at least the elements the kernel
will touch before anything is uploaded or launched.
"""

from __future__ import annotations

import numpy as np

from asdsl import _hip


def _numel(a) -> int:
    if type(a).__module__.startswith("torch"):
        return int(a.numel())
    return int(np.asarray(a).size)


def shape_of(a) -> tuple:
    if type(a).__module__.startswith("torch"):
        return tuple(a.shape)
    return tuple(np.shape(a))


def on_device(*arrays) -> bool:
    return any(_hip.is_device_tensor(a) for a in arrays if a is not None)


def new_output(shape, dtype, *like):
    """Output array for a returning wrapper: a device tensor when any input is
    one (the call stays asynchronous on the current stream), else numpy."""
    if on_device(*like):
        return _hip.empty_device(shape, dtype)
    return np.empty(shape, dtype)


class _Slot:
    __slots__ = ("array", "dtype", "n", "name", "is_output")

    def __init__(self, array, dtype, n, name, is_output):
        self.array, self.dtype, self.n, self.name, self.is_output = array, np.dtype(dtype), n, name, is_output


class _Scratch:
    __slots__ = ("n", "dtype")

    def __init__(self, n, dtype):
        self.n, self.dtype = n, np.dtype(dtype)


class DeviceCall:
    def __init__(self, fn: str):
        self.fn = fn

    def _check(self, a, dtype, n: int, name: str, is_output: bool) -> _Slot:
        if a is None:
            raise ValueError(f"{self.fn}: {name} is None")
        have = _numel(a)
        if have < n:
            raise ValueError(f"{self.fn}: {name} has {have} elements, needs {n}")
        if is_output:
            if type(a).__module__.startswith("torch"):
                import torch

                want = {np.dtype(np.float32): torch.float32, np.dtype(np.int8): torch.int8,
                        np.dtype(np.uint8): torch.uint8, np.dtype(np.int32): torch.int32,
                        np.dtype(np.uint32): torch.int32}[np.dtype(dtype)]
                if not a.is_cuda or a.dtype != want or not a.is_contiguous():
                    raise ValueError(f"{self.fn}: {name} must be a contiguous {np.dtype(dtype).name} device tensor")
            elif not isinstance(a, np.ndarray) or a.dtype != np.dtype(dtype) or not a.flags.c_contiguous:
                raise ValueError(f"{self.fn}: {name} must be a C-contiguous {np.dtype(dtype).name} array")
        return _Slot(a, dtype, n, name, is_output)

    def input(self, a, dtype, n: int, name: str) -> _Slot:
        return self._check(a, dtype, n, name, False)

    def output(self, a, dtype, n: int, name: str) -> _Slot:
        return self._check(a, dtype, n, name, True)

    def scratch(self, n: int, dtype) -> "_Scratch":
        """Device-only temporary of n elements (never copied back)."""
        return _Scratch(n, dtype)

    def run(self, entry: str, *args) -> None:
        keep, copyback, cargs = [], [], []
        for a in args:
            if isinstance(a, _Scratch):
                t = _hip.empty_device((max(a.n, 1),), a.dtype)
                keep.append(t)
                cargs.append(_hip.ptr(t))
                continue
            if not isinstance(a, _Slot):
                cargs.append(a)
                continue
            if a.is_output and _hip.is_device_tensor(a.array):
                cargs.append(_hip.ptr(a.array))
            elif a.is_output:
                t = _hip.empty_device((a.n,), a.dtype)
                keep.append(t)
                copyback.append((a.array, t, a.n))
                cargs.append(_hip.ptr(t))
            else:
                t = _hip.to_device(a.array, a.dtype)
                keep.append(t)
                cargs.append(_hip.ptr(t))
        _hip.call(entry, *cargs, _hip.stream_handle())
        for host, dev, n in copyback:
            host.reshape(-1)[:n] = dev.cpu().numpy().view(host.dtype)
