"""Minimal ctypes access to the HIP runtime that libattn_mi355x.so links
(/opt/rocm libamdhip64.so.7): device buffers, streams, events.

This is plumbing for the Python tests and the benchmark.  It deliberately
does not use PyTorch's device runtime: PyTorch wheels ship their own HIP
runtime, and two HIP runtimes in one process cannot both own the GPU.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_hip = None
_vp = ctypes.c_void_p


class HipError(RuntimeError):
    pass


def hip():
    global _hip
    if _hip is None:
        name = "libamdhip64.so.7"
        for cand in (name, os.path.join("/opt/rocm/lib", name)):
            try:
                _hip = ctypes.CDLL(cand)
                break
            except OSError:
                continue
        if _hip is None:
            raise HipError("cannot load libamdhip64.so.7")
        H = _hip
        H.hipGetErrorString.restype = ctypes.c_char_p
        H.hipGetErrorString.argtypes = [ctypes.c_int]
        H.hipMalloc.argtypes = [ctypes.POINTER(_vp), ctypes.c_size_t]
        H.hipFree.argtypes = [_vp]
        H.hipMemcpy.argtypes = [_vp, _vp, ctypes.c_size_t, ctypes.c_int]
        H.hipMemcpyAsync.argtypes = [_vp, _vp, ctypes.c_size_t, ctypes.c_int, _vp]
        H.hipMemset.argtypes = [_vp, ctypes.c_int, ctypes.c_size_t]
        H.hipDeviceSynchronize.argtypes = []
        H.hipGetDeviceCount.argtypes = [ctypes.POINTER(ctypes.c_int)]
        H.hipDeviceGetName.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int]
        H.hipStreamCreate.argtypes = [ctypes.POINTER(_vp)]
        H.hipStreamDestroy.argtypes = [_vp]
        H.hipStreamSynchronize.argtypes = [_vp]
        H.hipEventCreate.argtypes = [ctypes.POINTER(_vp)]
        H.hipEventDestroy.argtypes = [_vp]
        H.hipEventRecord.argtypes = [_vp, _vp]
        H.hipEventSynchronize.argtypes = [_vp]
        H.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), _vp, _vp]
        H.hipGetLastError.argtypes = []
        H.hipStreamBeginCapture.argtypes = [_vp, ctypes.c_int]
        H.hipStreamEndCapture.argtypes = [_vp, ctypes.POINTER(_vp)]
        H.hipGraphInstantiate.argtypes = [ctypes.POINTER(_vp), _vp, _vp, _vp, ctypes.c_size_t]
        H.hipGraphLaunch.argtypes = [_vp, _vp]
        H.hipGraphExecDestroy.argtypes = [_vp]
        H.hipGraphDestroy.argtypes = [_vp]
    return _hip


def check(err: int, what: str) -> None:
    if err != 0:
        msg = hip().hipGetErrorString(err).decode()
        raise HipError(f"{what}: hip error {err} ({msg})")


H2D, D2H, D2D = 1, 2, 3


def device_count() -> int:
    n = ctypes.c_int(0)
    if hip().hipGetDeviceCount(ctypes.byref(n)) != 0:
        return 0
    return n.value


def device_name(dev: int = 0) -> str:
    buf = ctypes.create_string_buffer(256)
    check(hip().hipDeviceGetName(buf, 256, dev), "hipDeviceGetName")
    return buf.value.decode()


def copy_d2d(dst: "DeviceArray", src: "DeviceArray", nbytes: int) -> None:
    """Device-to-device copy of nbytes (runs as the HIP runtime's copy kernel)."""
    assert nbytes <= min(dst.nbytes, src.nbytes)
    check(hip().hipMemcpy(_vp(dst.ptr), _vp(src.ptr), nbytes, D2D), "hipMemcpy D2D")


def copy_d2d_async(dst: "DeviceArray", src: "DeviceArray", nbytes: int, stream: "Stream") -> None:
    """Asynchronous device-to-device copy on `stream` (capturable into a graph)."""
    assert nbytes <= min(dst.nbytes, src.nbytes)
    check(hip().hipMemcpyAsync(_vp(dst.ptr), _vp(src.ptr), nbytes, D2D, _vp(stream.handle)),
          "hipMemcpyAsync D2D")


def synchronize() -> None:
    check(hip().hipDeviceSynchronize(), "hipDeviceSynchronize")


# ---------------------------------------------------------------- bf16 host conversion
def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bfloat16 bits (uint16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    if nan.any():
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------- buffers
class DeviceArray:
    """A device allocation with a shape and an element type ('f32' | 'bf16')."""

    def __init__(self, shape, dtype: str = "f32", fill=None):
        self.shape = tuple(int(s) for s in shape)
        self.dtype = dtype
        self.itemsize = 4 if dtype == "f32" else 2
        self.size = int(np.prod(self.shape)) if self.shape else 1
        self.nbytes = self.size * self.itemsize
        p = _vp()
        check(hip().hipMalloc(ctypes.byref(p), max(self.nbytes, 1)), "hipMalloc")
        self.base = p.value
        self.ptr = p.value
        self._owner = True
        if fill is not None:
            check(hip().hipMemset(_vp(self.ptr), fill, self.nbytes), "hipMemset")

    @classmethod
    def view(cls, base: "DeviceArray", offset_elems: int, shape, dtype=None):
        """Non-owning view at an element offset (for misalignment tests)."""
        obj = cls.__new__(cls)
        obj.shape = tuple(shape)
        obj.dtype = dtype or base.dtype
        obj.itemsize = 4 if obj.dtype == "f32" else 2
        obj.size = int(np.prod(obj.shape))
        obj.nbytes = obj.size * obj.itemsize
        obj.base = base.base
        obj.ptr = base.ptr + offset_elems * base.itemsize
        obj._owner = False
        obj._keep = base
        return obj

    @classmethod
    def from_numpy(cls, a: np.ndarray, dtype: str = "f32") -> "DeviceArray":
        """Upload float32 data; dtype 'bf16' rounds (RNE) on the host first.
        A uint16 array with dtype 'bf16' is taken as raw bf16 bits."""
        if dtype == "bf16":
            host = a if a.dtype == np.uint16 else f32_to_bf16_bits(a)
        else:
            host = np.ascontiguousarray(a, dtype=np.float32)
        host = np.ascontiguousarray(host)
        d = cls(a.shape, dtype)
        check(hip().hipMemcpy(_vp(d.ptr), host.ctypes.data_as(_vp), d.nbytes, H2D), "H2D")
        return d

    def upload(self, a: np.ndarray) -> None:
        host = f32_to_bf16_bits(a) if (self.dtype == "bf16" and a.dtype != np.uint16) else a
        host = np.ascontiguousarray(host, dtype=np.uint16 if self.dtype == "bf16" else np.float32)
        assert host.nbytes == self.nbytes
        check(hip().hipMemcpy(_vp(self.ptr), host.ctypes.data_as(_vp), self.nbytes, H2D), "H2D")

    def bits(self) -> np.ndarray:
        """Raw contents: float32 array, or uint16 bf16 bits."""
        out = np.empty(self.shape, dtype=np.float32 if self.dtype == "f32" else np.uint16)
        check(hip().hipMemcpy(out.ctypes.data_as(_vp), _vp(self.ptr), self.nbytes, D2H), "D2H")
        return out

    def numpy(self) -> np.ndarray:
        """Contents widened to float32."""
        b = self.bits()
        return b if self.dtype == "f32" else bf16_bits_to_f32(b)

    def fill_nan(self) -> None:
        check(hip().hipMemset(_vp(self.ptr), 0xFF, self.nbytes), "hipMemset")

    def free(self) -> None:
        if getattr(self, "_owner", False) and self.base:
            hip().hipFree(_vp(self.base))
            self.base = 0
            self._owner = False

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        s = _vp()
        check(hip().hipStreamCreate(ctypes.byref(s)), "hipStreamCreate")
        self.handle = s.value

    def synchronize(self) -> None:
        check(hip().hipStreamSynchronize(_vp(self.handle)), "hipStreamSynchronize")

    def destroy(self) -> None:
        if self.handle:
            hip().hipStreamDestroy(_vp(self.handle))
            self.handle = None


class Event:
    def __init__(self):
        e = _vp()
        check(hip().hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        self.handle = e.value

    def record(self, stream: Stream | None = None) -> None:
        check(hip().hipEventRecord(_vp(self.handle), _vp(stream.handle if stream else None)),
              "hipEventRecord")

    def synchronize(self) -> None:
        check(hip().hipEventSynchronize(_vp(self.handle)), "hipEventSynchronize")

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float(0)
        check(hip().hipEventElapsedTime(ctypes.byref(ms), _vp(self.handle), _vp(end.handle)),
              "hipEventElapsedTime")
        return ms.value

    def destroy(self) -> None:
        if self.handle:
            hip().hipEventDestroy(_vp(self.handle))
            self.handle = None


class Graph:
    """A HIP graph captured from the work `fn()` enqueues on `stream`
    (relaxed capture mode), instantiated for replay with launch()."""

    def __init__(self, stream: Stream, fn):
        H = hip()
        check(H.hipStreamBeginCapture(_vp(stream.handle), 2), "hipStreamBeginCapture")
        try:
            fn()
        finally:
            g = _vp()
            err = H.hipStreamEndCapture(_vp(stream.handle), ctypes.byref(g))
        check(err, "hipStreamEndCapture")
        self.graph = g.value
        e = _vp()
        check(H.hipGraphInstantiate(ctypes.byref(e), _vp(self.graph), None, None, 0),
              "hipGraphInstantiate")
        self.exec = e.value
        self.stream = stream

    def launch(self) -> None:
        check(hip().hipGraphLaunch(_vp(self.exec), _vp(self.stream.handle)), "hipGraphLaunch")

    def destroy(self) -> None:
        if self.exec:
            hip().hipGraphExecDestroy(_vp(self.exec))
            self.exec = None
        if self.graph:
            hip().hipGraphDestroy(_vp(self.graph))
            self.graph = None
