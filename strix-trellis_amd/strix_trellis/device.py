"""Device memory and streams through the HIP runtime itself (ctypes over
libamdhip64), for hosts without PyTorch.

The library's entry points take plain device pointers and HIP streams; this
module supplies them from NumPy:

    arr = device.DeviceArray.from_numpy(x)        # hipMalloc + H2D copy
    y = device.DeviceArray.empty((rows, n), np.float32)
    ... strix_gemv / strix_gemm through runtime ...
    out = y.numpy()                              # D2H copy (synchronous)

DeviceArray and Stream carry the small surface the runtime's descriptor
helpers read from a torch tensor or stream (``data_ptr()``, ``shape``,
``dtype``, ``numel()``, ``element_size()``, ``dim()``, ``is_contiguous()``,
``device``; ``cuda_stream``), so both kinds of buffers go through the same
calls.  Memory is freed by ``free()`` or when the object is collected.
"""
import ctypes as C
import os
from pathlib import Path

import numpy as np

_hip = None

HIP_MEMCPY_HOST_TO_DEVICE = 1
HIP_MEMCPY_DEVICE_TO_HOST = 2


class HipError(RuntimeError):
    def __init__(self, call, code):
        self.code = code
        super().__init__(f"{call} failed with hipError {code}")


def _candidates():
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    yield str(Path(rocm) / "lib" / "libamdhip64.so")
    yield "libamdhip64.so"


def hip():
    """The HIP runtime library, loaded once."""
    global _hip
    if _hip is None:
        last = None
        for name in _candidates():
            try:
                lib = C.CDLL(name)
                break
            except OSError as exc:
                last = exc
        else:
            raise RuntimeError(f"libamdhip64.so not found ({last})")
        vp, sz = C.c_void_p, C.c_size_t
        for fn, args in (("hipMalloc", [C.POINTER(vp), sz]), ("hipFree", [vp]),
                         ("hipMemcpy", [vp, vp, sz, C.c_int]),
                         ("hipMemcpyAsync", [vp, vp, sz, C.c_int, vp]),
                         ("hipStreamCreate", [C.POINTER(vp)]), ("hipStreamDestroy", [vp]),
                         ("hipStreamSynchronize", [vp]), ("hipDeviceSynchronize", []),
                         ("hipSetDevice", [C.c_int]), ("hipGetDevice", [C.POINTER(C.c_int)]),
                         ("hipGetDeviceCount", [C.POINTER(C.c_int)])):
            f = getattr(lib, fn)
            f.restype = C.c_int
            f.argtypes = args
        _hip = lib
    return _hip


def check(code, call):
    if code != 0:
        raise HipError(call, code)


def device_count():
    n = C.c_int(0)
    code = hip().hipGetDeviceCount(C.byref(n))
    return n.value if code == 0 else 0


def set_device(ordinal):
    check(hip().hipSetDevice(int(ordinal)), "hipSetDevice")


def current_device():
    d = C.c_int(0)
    check(hip().hipGetDevice(C.byref(d)), "hipGetDevice")
    return d.value


class _on_device:
    """Makes `ordinal` the current device for a block, then restores the previous one."""

    def __init__(self, ordinal):
        self.ordinal = int(ordinal)

    def __enter__(self):
        self.prev = current_device()
        if self.prev != self.ordinal:
            set_device(self.ordinal)

    def __exit__(self, *exc):
        if self.prev != self.ordinal:
            set_device(self.prev)


class Stream:
    """A HIP stream (``hipStreamCreate``) on device `device` (default: the current one)."""

    def __init__(self, device=None):
        h = C.c_void_p()
        with _on_device(current_device() if device is None else device):
            check(hip().hipStreamCreate(C.byref(h)), "hipStreamCreate")
        self.cuda_stream = h.value or 0

    def synchronize(self):
        check(hip().hipStreamSynchronize(C.c_void_p(self.cuda_stream or None)), "hipStreamSynchronize")

    def destroy(self):
        if self.cuda_stream:
            check(hip().hipStreamDestroy(C.c_void_p(self.cuda_stream)), "hipStreamDestroy")
            self.cuda_stream = 0


class DeviceArray:
    """A contiguous array in the memory of device `device` (one hipMalloc, 256-byte aligned)."""

    def __init__(self, shape, dtype, device=0):
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.device = int(device)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = C.c_void_p()
        if self.nbytes:
            with _on_device(self.device):
                check(hip().hipMalloc(C.byref(p), max(self.nbytes, 256)), "hipMalloc")
        self._ptr = p.value or 0

    # -- the surface the runtime's descriptor helpers read ----------------------
    def data_ptr(self):
        return self._ptr

    def numel(self):
        return int(np.prod(self.shape, dtype=np.int64))

    def element_size(self):
        return self.dtype.itemsize

    def dim(self):
        return len(self.shape)

    def is_contiguous(self):
        return True

    # -- construction and copies -------------------------------------------------
    @classmethod
    def empty(cls, shape, dtype=np.float32, device=0):
        return cls(shape, dtype, device)

    @classmethod
    def from_numpy(cls, a, dtype=None, device=0):
        a = np.ascontiguousarray(a, dtype=dtype)
        self = cls(a.shape, a.dtype, device)
        self.copy_from(a)
        return self

    def copy_from(self, a):
        """Synchronous host -> device copy of a NumPy array of the same size."""
        a = np.ascontiguousarray(a, dtype=self.dtype)
        if a.nbytes != self.nbytes:
            raise ValueError("size mismatch")
        if self.nbytes:
            check(hip().hipMemcpy(C.c_void_p(self._ptr), a.ctypes.data_as(C.c_void_p), self.nbytes,
                                  HIP_MEMCPY_HOST_TO_DEVICE), "hipMemcpy")
        return self

    def numpy(self):
        """Synchronous device -> host copy (waits for the device's work on it)."""
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            check(hip().hipMemcpy(out.ctypes.data_as(C.c_void_p), C.c_void_p(self._ptr), self.nbytes,
                                  HIP_MEMCPY_DEVICE_TO_HOST), "hipMemcpy")
        return out

    def free(self):
        if self._ptr:
            check(hip().hipFree(C.c_void_p(self._ptr)), "hipFree")
            self._ptr = 0

    def __del__(self):
        try:
            if self._ptr and _hip is not None:
                _hip.hipFree(C.c_void_p(self._ptr))
                self._ptr = 0
        except Exception:
            pass
