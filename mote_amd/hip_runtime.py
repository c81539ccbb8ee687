"""HIP events, graphs and device-to-device copies from the runtime that
``libmote_hip.so`` is linked against (the same ``libamdhip64.so.7`` instance,
so the library's streams are valid here).  Measurement and graph-capture
plumbing for the benchmark and the graph tests; the C ABI itself needs none of
it."""

from __future__ import annotations

import ctypes

from . import _ffi


class HipRuntime:
    """hipEvent / hipGraph / hipMemcpy entry points; every failing call raises
    :class:`mote_amd._ffi.HipError`."""

    CAPTURE_THREAD_LOCAL = 1  # hipStreamCaptureModeThreadLocal
    DEVICE_TO_DEVICE = 3      # hipMemcpyDeviceToDevice

    def __init__(self) -> None:
        _ffi.lib()  # loads libamdhip64.so.7 as a dependency first
        h = ctypes.CDLL("libamdhip64.so.7")
        P = ctypes.c_void_p
        h.hipEventCreate.argtypes = [ctypes.POINTER(P)]
        h.hipEventRecord.argtypes = [P, P]
        h.hipEventSynchronize.argtypes = [P]
        h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), P, P]
        h.hipEventDestroy.argtypes = [P]
        h.hipStreamBeginCapture.argtypes = [P, ctypes.c_int]
        h.hipStreamEndCapture.argtypes = [P, ctypes.POINTER(P)]
        h.hipGraphInstantiate.argtypes = [ctypes.POINTER(P), P, P, P, ctypes.c_size_t]
        h.hipGraphLaunch.argtypes = [P, P]
        h.hipGraphExecDestroy.argtypes = [P]
        h.hipGraphDestroy.argtypes = [P]
        h.hipMemcpy.argtypes = [P, P, ctypes.c_size_t, ctypes.c_int]
        h.hipStreamCreate.argtypes = [ctypes.POINTER(P)]
        h.hipDeviceSynchronize.argtypes = []
        self.h = h

    def foreign_stream(self) -> "ForeignStream":
        """A stream made by hipStreamCreate directly, as a caller's own
        stream would be (the library has reserved no scratch for it)."""
        s = ctypes.c_void_p()
        _ffi.check(self.h.hipStreamCreate(ctypes.byref(s)), "create stream")
        return ForeignStream(s.value)

    def device_synchronize(self) -> None:
        _ffi.check(self.h.hipDeviceSynchronize(), "device synchronize")

    def create(self) -> int:
        e = ctypes.c_void_p()
        _ffi.check(self.h.hipEventCreate(ctypes.byref(e)), "create event")
        return e.value

    def record(self, event: int, stream) -> None:
        _ffi.check(self.h.hipEventRecord(event, stream.handle), "record event")

    def elapsed_ms(self, start: int, stop: int) -> float:
        _ffi.check(self.h.hipEventSynchronize(stop), "synchronize event")
        ms = ctypes.c_float()
        _ffi.check(self.h.hipEventElapsedTime(ctypes.byref(ms), start, stop), "event elapsed time")
        return float(ms.value)

    def destroy(self, event: int) -> None:
        _ffi.check(self.h.hipEventDestroy(event), "destroy event")

    def capture(self, stream, body) -> int:
        """Records the launches `body()` enqueues on `stream` into an
        executable graph (nothing runs during capture)."""
        _ffi.check(self.h.hipStreamBeginCapture(stream.handle, self.CAPTURE_THREAD_LOCAL), "begin capture")
        try:
            body()
        finally:
            graph = ctypes.c_void_p()
            status = self.h.hipStreamEndCapture(stream.handle, ctypes.byref(graph))
        _ffi.check(status, "end capture")
        exe = ctypes.c_void_p()
        status = self.h.hipGraphInstantiate(ctypes.byref(exe), graph, None, None, 0)
        self.h.hipGraphDestroy(graph)
        _ffi.check(status, "instantiate graph")
        return exe.value

    def launch_graph(self, exe: int, stream) -> None:
        _ffi.check(self.h.hipGraphLaunch(exe, stream.handle), "launch graph")

    def destroy_graph(self, exe: int) -> None:
        _ffi.check(self.h.hipGraphExecDestroy(exe), "destroy graph")

    def copy_device_to_device(self, dst: int, src: int, nbytes: int) -> None:
        _ffi.check(self.h.hipMemcpy(dst, src, nbytes, self.DEVICE_TO_DEVICE), "device-to-device copy")


class ForeignStream:
    """A HIP stream the library did not create; close() hands it to
    mote_hip_stream_destroy, which also parks the scratch the library kept
    for it."""

    def __init__(self, handle: int) -> None:
        self.handle = handle

    def synchronize(self) -> None:
        _ffi.check(_ffi.lib().mote_hip_stream_synchronize(self.handle), "synchronize stream")

    def close(self) -> None:
        if self.handle:
            _ffi.check(_ffi.lib().mote_hip_stream_destroy(self.handle), "destroy stream")
            self.handle = 0
