"""Device memory, streams and events over the C ABI (no torch involved).

The GPU process uses only libperegrine_hip.so's runtime entry points for
memory (hipMalloc / hipMemcpy underneath), so a single HIP runtime is loaded.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import call, lib

_initialized = False


def device_count() -> int:
    n = C.c_int(0)
    rc = lib.prg_hip_device_count(C.byref(n))
    return n.value if rc == 0 else 0


def init(ordinal: int = 0) -> None:
    global _initialized
    if not _initialized:
        call("prg_hip_device_init", ordinal)
        _initialized = True


def device_name() -> str:
    buf = C.create_string_buffer(256)
    call("prg_hip_device_name", buf, 256)
    return buf.value.decode()


def synchronize() -> None:
    call("prg_hip_device_synchronize")


class DeviceArray:
    """A device allocation with a numpy dtype and shape. Frees on close/del."""

    def __init__(self, shape, dtype) -> None:
        init()
        self.shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = C.c_void_p(0)
        call("prg_hip_alloc_device", C.byref(p), C.c_size_t(self.nbytes))
        self._ptr = p.value or 0

    @property
    def ptr(self) -> int:
        return self._ptr

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "DeviceArray":
        a = np.ascontiguousarray(a)
        d = cls(a.shape, a.dtype)
        d.upload(a)
        return d

    @classmethod
    def zeros(cls, shape, dtype) -> "DeviceArray":
        d = cls(shape, dtype)
        d.fill_zero()
        return d

    def upload(self, a: np.ndarray, stream=None) -> None:
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes, (a.nbytes, self.nbytes)
        if self.nbytes:
            call("prg_hip_memcpy", C.c_void_p(self._ptr), a.ctypes.data_as(C.c_void_p),
                 C.c_size_t(self.nbytes), 0, stream, 1)

    def numpy(self, stream=None) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            call("prg_hip_memcpy", out.ctypes.data_as(C.c_void_p), C.c_void_p(self._ptr),
                 C.c_size_t(self.nbytes), 1, stream, 1)
        return out

    def fill_zero(self, stream=None) -> None:
        call("prg_hip_memset_device", C.c_void_p(self._ptr), 0, C.c_size_t(self.nbytes), stream)
        if stream is None:
            synchronize()

    def close(self) -> None:
        if self._ptr:
            lib.prg_hip_free_device(C.c_void_p(self._ptr))
            self._ptr = 0

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass


class Stream:
    def __init__(self) -> None:
        init()
        p = C.c_void_p(0)
        call("prg_hip_stream_create", C.byref(p))
        self.handle = p.value

    def synchronize(self) -> None:
        call("prg_hip_stream_synchronize", C.c_void_p(self.handle))

    def close(self) -> None:
        if self.handle:
            lib.prg_hip_stream_destroy(C.c_void_p(self.handle))
            self.handle = None


class Event:
    def __init__(self) -> None:
        init()
        p = C.c_void_p(0)
        call("prg_hip_event_create", C.byref(p))
        self.handle = p.value

    def record(self, stream=None) -> None:
        call("prg_hip_event_record", C.c_void_p(self.handle), stream)

    def elapsed_ms(self, end: "Event") -> float:
        ms = C.c_float(0.0)
        call("prg_hip_event_elapsed_ms", C.c_void_p(self.handle), C.c_void_p(end.handle), C.byref(ms))
        return float(ms.value)

    def close(self) -> None:
        if self.handle:
            lib.prg_hip_event_destroy(C.c_void_p(self.handle))
            self.handle = None


class Graph:
    """Ops issued on `stream` inside `with Graph.capture(stream) as g:` are
    recorded once and replayed by g.launch() (prg_hip_graph_*)."""

    def __init__(self, stream: Stream) -> None:
        self.stream = stream
        self.handle = None

    @classmethod
    def capture(cls, stream: Stream) -> "Graph":
        return cls(stream)

    def __enter__(self) -> "Graph":
        call("prg_hip_graph_begin", C.c_void_p(self.stream.handle))
        return self

    def __exit__(self, exc_type, exc, tb) -> None:
        h = C.c_void_p(0)
        rc = lib.prg_hip_graph_end(C.c_void_p(self.stream.handle), C.byref(h))
        if exc_type is None:
            if rc != 0:
                raise RuntimeError(f"prg_hip_graph_end failed ({rc}): {lib.prg_last_error().decode()}")
            self.handle = h.value

    def launch(self) -> None:
        call("prg_hip_graph_launch", C.c_void_p(self.handle), C.c_void_p(self.stream.handle))

    def close(self) -> None:
        if self.handle:
            lib.prg_hip_graph_destroy(C.c_void_p(self.handle))
            self.handle = None


def ptr(x) -> C.c_void_p:
    """Device pointer argument for a DeviceArray, int or None."""
    if x is None:
        return C.c_void_p(0)
    if isinstance(x, DeviceArray):
        return C.c_void_p(x.ptr)
    return C.c_void_p(int(x))
