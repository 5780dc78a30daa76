"""Minimal ctypes view of the HIP runtime: device memory, copies, streams and
events. It is plumbing for tests and the benchmark (it imports in well under a
second, unlike torch), not part of the MoE path itself."""
import ctypes
import os

import numpy as np

_ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
_hip = ctypes.CDLL(os.path.join(_ROCM, "lib", "libamdhip64.so"), mode=ctypes.RTLD_GLOBAL)

_vp = ctypes.c_void_p
_sz = ctypes.c_size_t

_hip.hipGetErrorString.restype = ctypes.c_char_p
_hip.hipGetErrorString.argtypes = [ctypes.c_int]
for name, args in [
    ("hipMalloc", [ctypes.POINTER(_vp), _sz]),
    ("hipFree", [_vp]),
    ("hipMemcpy", [_vp, _vp, _sz, ctypes.c_int]),
    ("hipMemcpyAsync", [_vp, _vp, _sz, ctypes.c_int, _vp]),
    ("hipMemset", [_vp, ctypes.c_int, _sz]),
    ("hipDeviceSynchronize", []),
    ("hipGetDeviceCount", [ctypes.POINTER(ctypes.c_int)]),
    ("hipSetDevice", [ctypes.c_int]),
    ("hipStreamCreate", [ctypes.POINTER(_vp)]),
    ("hipStreamDestroy", [_vp]),
    ("hipStreamSynchronize", [_vp]),
    ("hipEventCreate", [ctypes.POINTER(_vp)]),
    ("hipEventDestroy", [_vp]),
    ("hipEventRecord", [_vp, _vp]),
    ("hipEventSynchronize", [_vp]),
    ("hipEventElapsedTime", [ctypes.POINTER(ctypes.c_float), _vp, _vp]),
    ("hipMemGetInfo", [ctypes.POINTER(_sz), ctypes.POINTER(_sz)]),
    ("hipHostMalloc", [ctypes.POINTER(_vp), _sz, ctypes.c_uint]),
    ("hipHostFree", [_vp]),
    ("hipStreamBeginCapture", [_vp, ctypes.c_int]),
    ("hipStreamEndCapture", [_vp, ctypes.POINTER(_vp)]),
    ("hipGraphInstantiate", [ctypes.POINTER(_vp), _vp, _vp, ctypes.c_char_p, _sz]),
    ("hipGraphLaunch", [_vp, _vp]),
    ("hipGraphExecDestroy", [_vp]),
    ("hipGraphDestroy", [_vp]),
]:
    fn = getattr(_hip, name)
    fn.argtypes = args
    fn.restype = ctypes.c_int

H2D, D2H, D2D = 1, 2, 3


class HipError(RuntimeError):
    pass


def check(rc, what=""):
    if rc != 0:
        raise HipError(f"{what}: {_hip.hipGetErrorString(rc).decode()} ({rc})")


def device_count():
    n = ctypes.c_int(0)
    rc = _hip.hipGetDeviceCount(ctypes.byref(n))
    return n.value if rc == 0 else 0


def synchronize():
    check(_hip.hipDeviceSynchronize(), "hipDeviceSynchronize")


def mem_info():
    free, total = _sz(0), _sz(0)
    check(_hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)), "hipMemGetInfo")
    return free.value, total.value


class DeviceBuffer:
    """An owned device allocation of `nbytes`."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = _vp()
        check(_hip.hipMalloc(ctypes.byref(p), max(self.nbytes, 16)), f"hipMalloc({self.nbytes})")
        self.ptr = p.value

    @classmethod
    def from_array(cls, arr):
        arr = np.ascontiguousarray(arr)
        b = cls(arr.nbytes)
        b.upload(arr)
        return b

    def upload(self, arr, offset=0):
        arr = np.ascontiguousarray(arr)
        assert offset + arr.nbytes <= self.nbytes
        check(_hip.hipMemcpy(_vp(self.ptr + offset), arr.ctypes.data_as(_vp), arr.nbytes, H2D), "H2D")

    def download(self, dtype, count=None, offset=0):
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        out = np.empty(count, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes
        check(_hip.hipMemcpy(out.ctypes.data_as(_vp), _vp(self.ptr + offset), out.nbytes, D2H), "D2H")
        return out

    def zero(self):
        check(_hip.hipMemset(_vp(self.ptr), 0, self.nbytes), "hipMemset")

    def free(self):
        if self.ptr:
            _hip.hipFree(_vp(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class HostBuffer:
    """An owned pinned host allocation (hipHostMalloc) of `nbytes`."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = _vp()
        check(_hip.hipHostMalloc(ctypes.byref(p), max(self.nbytes, 16), 0), f"hipHostMalloc({self.nbytes})")
        self.ptr = p.value

    def view(self, dtype=np.uint8, count=None, offset=0):
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dtype.itemsize
        buf = (ctypes.c_uint8 * (count * dtype.itemsize)).from_address(self.ptr + offset)
        return np.frombuffer(buf, dtype=dtype, count=count)

    def free(self):
        if self.ptr:
            _hip.hipHostFree(_vp(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def copy_d2h_ptr(dst_host, src_dev, nbytes):
    check(_hip.hipMemcpy(_vp(dst_host), _vp(src_dev), nbytes, D2H), "D2H")


def download_ptr(ptr, dtype, count):
    out = np.empty(count, dtype=np.dtype(dtype))
    check(_hip.hipMemcpy(out.ctypes.data_as(_vp), _vp(ptr), out.nbytes, D2H), "D2H")
    return out


def copy_d2d(dst, src, nbytes, stream=None):
    check(_hip.hipMemcpyAsync(_vp(dst), _vp(src), nbytes, D2D, _vp(stream or 0)), "D2D")


class Stream:
    def __init__(self):
        p = _vp()
        check(_hip.hipStreamCreate(ctypes.byref(p)), "hipStreamCreate")
        self.handle = p.value

    def synchronize(self):
        check(_hip.hipStreamSynchronize(_vp(self.handle)), "hipStreamSynchronize")

    def destroy(self):
        if self.handle:
            _hip.hipStreamDestroy(_vp(self.handle))
            self.handle = None


class Event:
    def __init__(self):
        p = _vp()
        check(_hip.hipEventCreate(ctypes.byref(p)), "hipEventCreate")
        self.handle = p.value

    def record(self, stream=None):
        check(_hip.hipEventRecord(_vp(self.handle), _vp(stream.handle if stream else 0)), "hipEventRecord")

    def synchronize(self):
        check(_hip.hipEventSynchronize(_vp(self.handle)), "hipEventSynchronize")

    def elapsed_ms(self, end):
        ms = ctypes.c_float(0)
        check(_hip.hipEventElapsedTime(ctypes.byref(ms), _vp(self.handle), _vp(end.handle)), "elapsed")
        return ms.value


class Graph:
    """A HIP graph captured from one stream (global capture mode): the work
    enqueued between begin() and end() is recorded, not run; launch() replays
    it on a stream."""

    def __init__(self, stream):
        self.stream = stream
        self.graph = None
        self.exec = None

    def begin(self):
        check(_hip.hipStreamBeginCapture(_vp(self.stream.handle), 0), "hipStreamBeginCapture")

    def end(self):
        g = _vp()
        check(_hip.hipStreamEndCapture(_vp(self.stream.handle), ctypes.byref(g)), "hipStreamEndCapture")
        self.graph = g.value
        if self.graph:
            e = _vp()
            check(_hip.hipGraphInstantiate(ctypes.byref(e), _vp(self.graph), None, None, 0), "hipGraphInstantiate")
            self.exec = e.value

    def launch(self):
        check(_hip.hipGraphLaunch(_vp(self.exec), _vp(self.stream.handle)), "hipGraphLaunch")

    def destroy(self):
        if self.exec:
            _hip.hipGraphExecDestroy(_vp(self.exec))
            self.exec = None
        if self.graph:
            _hip.hipGraphDestroy(_vp(self.graph))
            self.graph = None
