"""Minimal ctypes binding of the HIP runtime (libamdhip64): device buffers, streams, events.

Plumbing for tests and benchmarks that drive libternix_hip.so through its C-ABI with device
pointers.  No PyTorch: the library's entry points take plain device pointers and a hipStream_t.
"""
import ctypes
import ctypes.util
import os

import numpy as np

H2D, D2H, D2D = 1, 2, 3

_hip = None


def _load():
    global _hip
    if _hip is not None:
        return _hip
    cands = []
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cands += [os.path.join(rocm, "lib", "libamdhip64.so"), "libamdhip64.so", "libamdhip64.so.7"]
    found = ctypes.util.find_library("amdhip64")
    if found:
        cands.append(found)
    last = None
    for c in cands:
        try:
            _hip = ctypes.CDLL(c)
            break
        except OSError as e:
            last = e
    if _hip is None:
        raise OSError(f"HIP runtime (libamdhip64.so) not found: {last}")
    v, p, sz, i, f = ctypes.c_void_p, ctypes.POINTER, ctypes.c_size_t, ctypes.c_int, ctypes.c_float
    _hip.hipMalloc.argtypes = [p(v), sz]
    _hip.hipFree.argtypes = [v]
    _hip.hipMemcpy.argtypes = [v, v, sz, i]
    _hip.hipMemcpyAsync.argtypes = [v, v, sz, i, v]
    _hip.hipDeviceSynchronize.argtypes = []
    _hip.hipGetDeviceCount.argtypes = [p(i)]
    _hip.hipSetDevice.argtypes = [i]
    _hip.hipStreamCreate.argtypes = [p(v)]
    _hip.hipStreamDestroy.argtypes = [v]
    _hip.hipStreamSynchronize.argtypes = [v]
    _hip.hipEventCreate.argtypes = [p(v)]
    _hip.hipEventDestroy.argtypes = [v]
    _hip.hipEventRecord.argtypes = [v, v]
    _hip.hipEventSynchronize.argtypes = [v]
    _hip.hipEventElapsedTime.argtypes = [p(f), v, v]
    _hip.hipGetErrorString.argtypes = [i]
    _hip.hipGetErrorString.restype = ctypes.c_char_p
    _hip.hipDeviceGetAttribute.argtypes = [p(i), i, i]
    _hip.hipDeviceGetName.argtypes = [ctypes.c_char_p, i, i]
    _hip.hipStreamBeginCapture.argtypes = [v, i]
    _hip.hipStreamEndCapture.argtypes = [v, p(v)]
    _hip.hipGraphInstantiate.argtypes = [p(v), v, v, v, sz]
    _hip.hipGraphLaunch.argtypes = [v, v]
    _hip.hipGraphExecDestroy.argtypes = [v]
    _hip.hipGraphDestroy.argtypes = [v]
    return _hip


class HipError(RuntimeError):
    pass


def check(status, what=""):
    if status != 0:
        msg = _load().hipGetErrorString(status)
        raise HipError(f"HIP error {status} ({msg.decode() if msg else '?'}) in {what}")


def device_count():
    try:
        hip = _load()
    except OSError:
        return 0
    n = ctypes.c_int(0)
    if hip.hipGetDeviceCount(ctypes.byref(n)) != 0:
        return 0
    return n.value


def synchronize():
    check(_load().hipDeviceSynchronize(), "hipDeviceSynchronize")


def device_name(dev=0):
    buf = ctypes.create_string_buffer(256)
    check(_load().hipDeviceGetName(buf, 256, dev), "hipDeviceGetName")
    return buf.value.decode(errors="replace")


def device_attribute(attr, dev=0):
    out = ctypes.c_int(0)
    check(_load().hipDeviceGetAttribute(ctypes.byref(out), attr, dev), "hipDeviceGetAttribute")
    return out.value


# hipDeviceAttribute_t values used here (hip/hip_runtime_api.h, ROCm 7).
ATTR_CLOCK_RATE_KHZ = 5
ATTR_MULTIPROCESSOR_COUNT = 63


class DeviceBuffer:
    """An owning device allocation of `nbytes` bytes."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = ctypes.c_void_p()
        check(_load().hipMalloc(ctypes.byref(self.ptr), max(self.nbytes, 16)), f"hipMalloc({self.nbytes})")

    @classmethod
    def from_array(cls, arr):
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.upload(arr)
        return buf

    @property
    def value(self):
        return self.ptr.value

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        if arr.nbytes:
            check(_load().hipMemcpy(self.ptr, arr.ctypes.data_as(ctypes.c_void_p), arr.nbytes, H2D), "hipMemcpy H2D")

    def download(self, dtype, shape):
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        if out.nbytes:
            check(_load().hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), self.ptr, out.nbytes, D2H), "hipMemcpy D2H")
        return out

    def fill_from(self, arr):
        self.upload(arr)

    def free(self):
        if self.ptr and self.ptr.value:
            _load().hipFree(self.ptr)
            self.ptr = ctypes.c_void_p()

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    """A hipStream_t at default priority."""

    def __init__(self):
        self.handle = ctypes.c_void_p()
        check(_load().hipStreamCreate(ctypes.byref(self.handle)), "hipStreamCreate")

    def synchronize(self):
        check(_load().hipStreamSynchronize(self.handle), "hipStreamSynchronize")

    def __del__(self):
        try:
            if self.handle.value:
                _load().hipStreamDestroy(self.handle)
        except Exception:
            pass


class Event:
    def __init__(self):
        self.handle = ctypes.c_void_p()
        check(_load().hipEventCreate(ctypes.byref(self.handle)), "hipEventCreate")

    def record(self, stream=None):
        check(_load().hipEventRecord(self.handle, stream.handle if stream else None), "hipEventRecord")

    def synchronize(self):
        check(_load().hipEventSynchronize(self.handle), "hipEventSynchronize")

    def elapsed_ms(self, end):
        out = ctypes.c_float(0)
        check(_load().hipEventElapsedTime(ctypes.byref(out), self.handle, end.handle), "hipEventElapsedTime")
        return out.value

    def __del__(self):
        try:
            if self.handle.value:
                _load().hipEventDestroy(self.handle)
        except Exception:
            pass


class Graph:
    """Captures the work a callable enqueues on `stream` into a hipGraph; replay with launch()."""

    def __init__(self, stream, fn):
        hip = _load()
        self.graph = ctypes.c_void_p()
        self.exec = ctypes.c_void_p()
        check(hip.hipStreamBeginCapture(stream.handle, 0), "hipStreamBeginCapture")
        try:
            fn()
        finally:
            check(hip.hipStreamEndCapture(stream.handle, ctypes.byref(self.graph)), "hipStreamEndCapture")
        check(hip.hipGraphInstantiate(ctypes.byref(self.exec), self.graph, None, None, 0), "hipGraphInstantiate")
        self.stream = stream

    def launch(self):
        check(_load().hipGraphLaunch(self.exec, self.stream.handle), "hipGraphLaunch")

    def __del__(self):
        try:
            hip = _load()
            if self.exec.value:
                hip.hipGraphExecDestroy(self.exec)
            if self.graph.value:
                hip.hipGraphDestroy(self.graph)
        except Exception:
            pass
