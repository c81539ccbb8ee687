"""Device memory and streams through the library's own runtime wrappers
(``mote_hip_malloc`` / ``mote_hip_memcpy_*`` / ``mote_hip_stream_*``), the
ownership model of ``crates/mote-backend-hip/src/storage.rs:8-96``: a buffer
owns one ``hipMalloc`` allocation (at least one byte, so even an empty tensor
has a non-null pointer), uploads and reads back synchronously, and frees on
``free()`` / garbage collection.  Every runtime status is checked: ``free()``
and ``close()`` raise :class:`mote_amd._ffi.HipError` when the runtime
refuses, and forget the handle only once the runtime has released it (garbage
collection, which cannot raise, reports a failure on stderr)."""

from __future__ import annotations

import ctypes
import sys

import numpy as np

from ._ffi import check, lib


class Stream:
    """A HIP stream created by ``mote_hip_stream_create``."""

    def __init__(self) -> None:
        handle = ctypes.c_void_p()
        check(lib().mote_hip_stream_create(ctypes.byref(handle)), "create stream")
        self.handle: int = handle.value

    def synchronize(self) -> None:
        check(lib().mote_hip_stream_synchronize(self.handle), "synchronize stream")

    def close(self) -> None:
        if self.handle:
            check(lib().mote_hip_stream_synchronize(self.handle), "synchronize stream")
            check(lib().mote_hip_stream_destroy(self.handle), "destroy stream")
            self.handle = 0

    def __del__(self) -> None:  # pragma: no cover - best effort
        try:
            self.close()
        except Exception as e:
            print(f"mote_amd: stream not released: {e}", file=sys.stderr)


class DeviceBuffer:
    """One device allocation of ``nbytes`` bytes (>= 1 allocated)."""

    def __init__(self, nbytes: int) -> None:
        ptr = ctypes.c_void_p()
        check(lib().mote_hip_malloc(ctypes.byref(ptr), max(int(nbytes), 1)), "allocate device storage")
        self.ptr: int = ptr.value
        self.nbytes = int(nbytes)

    @classmethod
    def from_array(cls, array: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(array)
        buf = cls(a.nbytes)
        buf.upload(a)
        return buf

    def upload(self, array: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(array)
        if offset + a.nbytes > self.nbytes:
            raise ValueError("upload exceeds the buffer")
        if a.nbytes:
            check(
                lib().mote_hip_memcpy_host_to_device(self.ptr + offset, a.ctypes.data, a.nbytes),
                "upload device storage",
            )

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dt = np.dtype(dtype)
        n = (self.nbytes - offset) // dt.itemsize if count is None else int(count)
        out = np.empty(n, dtype=dt)
        if out.nbytes:
            check(
                lib().mote_hip_memcpy_device_to_host(out.ctypes.data, self.ptr + offset, out.nbytes),
                "read device storage",
            )
        return out

    def free(self) -> None:
        if self.ptr:
            check(lib().mote_hip_free(self.ptr), "free device storage")
            self.ptr = 0

    def __del__(self) -> None:  # pragma: no cover - best effort
        try:
            self.free()
        except Exception as e:
            print(f"mote_amd: device buffer not released: {e}", file=sys.stderr)


def device_count() -> int:
    count = ctypes.c_int(0)
    status = lib().mote_hip_get_device_count(ctypes.byref(count))
    return count.value if status == 0 else 0


def memory_info() -> tuple[int, int]:
    free = ctypes.c_size_t(0)
    total = ctypes.c_size_t(0)
    check(lib().mote_hip_mem_get_info(ctypes.byref(free), ctypes.byref(total)), "query device memory info")
    return free.value, total.value
