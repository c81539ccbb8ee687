"""GGUF model files as memory-mapped weight storage, uploaded verbatim.

The reference plans GGUF as a loader in front of its tensor model, not as the
tensor model itself: the file is memory-mapped, each weight is a byte range of
it, and weights are later copied into GPU storage (docs/tensor-design.md:
443-459, docs/roadmap.md:88).  This module is that loader for the formats the
path computes on: it parses the GGUF header (versions 2 and 3, little endian),
describes every tensor with the reference's span rules
(crates/mote-types/src/tensor_desc.rs:52-101: the last dimension is the
contiguous quantized row, it must hold whole blocks, every outer dimension
counts whole rows; the block geometry of crates/mote-types/src/lib.rs:39-74),
and returns a tensor's bytes as a read-only view of the mapping or uploads
them unchanged into a :class:`~mote_amd.device.DeviceBuffer` (as
``HipStorage::from_bytes`` takes GGML bytes verbatim,
crates/mote-backend-hip/src/storage.rs:15-45).

GGUF layout (the published format of the GGML project): magic ``GGUF``,
``u32`` version, ``u64`` tensor count, ``u64`` metadata count; metadata
entries ``(string key, u32 type, value)``; tensor infos ``(string name, u32
n_dims, u64 ne[n_dims], u32 ggml_type, u64 offset)`` with ``ne[0]`` the
innermost (contiguous) dimension and offsets relative to the data section,
which starts at the first multiple of ``general.alignment`` (default 32)
after the tensor infos.  Strings are ``u64`` length + UTF-8 bytes.
"""

from __future__ import annotations

import mmap
import os
import struct
from dataclasses import dataclass

import numpy as np

MAGIC = b"GGUF"
DEFAULT_ALIGNMENT = 32

# ggml tensor types this path knows: (encoding name, block elements, block bytes).
# Plain types use one-element "blocks" of their element size.
GGML_TYPES = {
    0: ("f32", 1, 4),
    1: ("f16", 1, 2),
    2: ("q4_0", 32, 18),
    8: ("q8_0", 32, 34),
    12: ("q4_k", 256, 144),
    14: ("q6_k", 256, 210),
}

# metadata value types
_U8, _I8, _U16, _I16, _U32, _I32, _F32, _BOOL, _STR, _ARR, _U64, _I64, _F64 = range(13)
_SCALARS = {
    _U8: "<B", _I8: "<b", _U16: "<H", _I16: "<h", _U32: "<I", _I32: "<i", _F32: "<f",
    _BOOL: "<?", _U64: "<Q", _I64: "<q", _F64: "<d",
}


class GGUFError(ValueError):
    """A malformed or unsupported GGUF file (the message names the cause)."""


@dataclass(frozen=True)
class TensorInfo:
    """One tensor of the file: ``shape`` outermost first (``[N, K]`` for a
    weight matrix whose rows are K long), ``offset`` absolute in the file,
    ``nbytes`` its span by the reference's rules."""

    name: str
    shape: tuple[int, ...]
    ggml_type: int
    encoding: str
    offset: int
    nbytes: int

    @property
    def quantized(self) -> bool:
        return GGML_TYPES[self.ggml_type][1] > 1


def span_bytes(shape: tuple[int, ...], ggml_type: int) -> int:
    """Byte span of a contiguous tensor (crates/mote-types/src/tensor_desc.rs:
    52-101): plain types numel * size; quantized types need a non-scalar shape
    whose last dimension is a whole number of blocks."""
    if ggml_type not in GGML_TYPES:
        raise GGUFError(f"unsupported ggml tensor type {ggml_type}")
    encoding, block_elements, block_bytes = GGML_TYPES[ggml_type]
    numel = 1
    for d in shape:
        numel *= d
    if block_elements == 1:
        return numel * block_bytes
    if not shape:
        raise GGUFError(f"quantized {encoding} tensor with a scalar shape")
    row = shape[-1]
    if row % block_elements:
        raise GGUFError(f"{encoding} row of {row} elements is not a whole number of "
                        f"{block_elements}-element blocks")
    if numel == 0:
        return 0
    return (numel // row) * (row // block_elements) * block_bytes


class _Reader:
    def __init__(self, buf, size: int) -> None:
        self.buf, self.size, self.pos = buf, size, 0

    def take(self, n: int) -> bytes:
        if n < 0 or self.pos + n > self.size:
            raise GGUFError(f"truncated file: {n} bytes needed at offset {self.pos}, size {self.size}")
        out = bytes(self.buf[self.pos:self.pos + n])
        self.pos += n
        return out

    def scalar(self, fmt: str):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        n = self.scalar("<Q")
        try:
            return self.take(n).decode("utf-8")
        except UnicodeDecodeError as e:
            raise GGUFError(f"string at offset {self.pos - n} is not UTF-8") from e

    def value(self, vtype: int, depth: int = 0):
        if vtype in _SCALARS:
            return self.scalar(_SCALARS[vtype])
        if vtype == _STR:
            return self.string()
        if vtype == _ARR:
            if depth > 8:
                raise GGUFError("metadata arrays nested too deeply")
            etype = self.scalar("<I")
            count = self.scalar("<Q")
            if count > self.size:
                raise GGUFError(f"metadata array of {count} elements exceeds the file")
            return [self.value(etype, depth + 1) for _ in range(count)]
        raise GGUFError(f"unknown metadata value type {vtype}")


class GGUFFile:
    """A memory-mapped GGUF file: ``metadata`` (dict), ``tensors`` (name ->
    :class:`TensorInfo`, file order), ``version``, ``alignment``,
    ``data_offset``.  Close it (or use it as a context manager) to release the
    mapping; a view returned by :meth:`tensor_bytes` that is still alive then
    keeps the mapping open until the view itself is dropped."""

    def __init__(self, path: str | os.PathLike) -> None:
        self.path = os.fspath(path)
        self._file = open(self.path, "rb")
        size = os.fstat(self._file.fileno()).st_size
        if size == 0:
            self._file.close()
            raise GGUFError("empty file")
        self._map = mmap.mmap(self._file.fileno(), 0, access=mmap.ACCESS_READ)
        try:
            self._parse(size)
        except Exception:
            self.close()
            raise

    def _parse(self, size: int) -> None:
        r = _Reader(self._map, size)
        if r.take(4) != MAGIC:
            raise GGUFError("not a GGUF file (bad magic)")
        self.version = r.scalar("<I")
        if self.version not in (2, 3):
            raise GGUFError(f"unsupported GGUF version {self.version}")
        n_tensors = r.scalar("<Q")
        n_kv = r.scalar("<Q")
        if n_tensors > size or n_kv > size:
            raise GGUFError("tensor or metadata count exceeds the file")
        self.metadata: dict = {}
        for _ in range(n_kv):
            key = r.string()
            self.metadata[key] = r.value(r.scalar("<I"))
        self.alignment = int(self.metadata.get("general.alignment", DEFAULT_ALIGNMENT))
        if self.alignment <= 0 or self.alignment & (self.alignment - 1):
            raise GGUFError(f"general.alignment {self.alignment} is not a power of two")
        infos = []
        for _ in range(n_tensors):
            name = r.string()
            n_dims = r.scalar("<I")
            if n_dims > 8:
                raise GGUFError(f"tensor {name!r} has {n_dims} dimensions")
            ne = [r.scalar("<Q") for _ in range(n_dims)]
            ggml_type = r.scalar("<I")
            offset = r.scalar("<Q")
            infos.append((name, tuple(reversed(ne)), ggml_type, offset))
        self.data_offset = -(-r.pos // self.alignment) * self.alignment
        self.tensors: dict[str, TensorInfo] = {}
        for name, shape, ggml_type, rel in infos:
            if name in self.tensors:
                raise GGUFError(f"duplicate tensor name {name!r}")
            if ggml_type not in GGML_TYPES:
                raise GGUFError(f"tensor {name!r}: unsupported ggml tensor type {ggml_type}")
            if rel % self.alignment:
                raise GGUFError(f"tensor {name!r}: offset {rel} is not {self.alignment}-byte aligned")
            try:
                nbytes = span_bytes(shape, ggml_type)
            except GGUFError as e:
                raise GGUFError(f"tensor {name!r}: {e}") from None
            start = self.data_offset + rel
            if start + nbytes > size:
                raise GGUFError(f"tensor {name!r} ({nbytes} bytes at {start}) extends past the end "
                                f"of the file ({size} bytes)")
            self.tensors[name] = TensorInfo(name, shape, ggml_type, GGML_TYPES[ggml_type][0], start, nbytes)

    def tensor_bytes(self, name: str) -> np.ndarray:
        """The tensor's bytes as a read-only uint8 view of the mapping."""
        info = self._info(name)
        return np.frombuffer(self._map, dtype=np.uint8, count=info.nbytes, offset=info.offset)

    def upload(self, name: str):
        """Copies the tensor's bytes unchanged into new device storage and
        returns ``(DeviceBuffer, TensorInfo)``."""
        from .device import DeviceBuffer  # device memory only when asked for

        info = self._info(name)
        buf = DeviceBuffer(info.nbytes)
        if info.nbytes:
            buf.upload(self.tensor_bytes(name))
        return buf, info

    def _info(self, name: str) -> TensorInfo:
        try:
            return self.tensors[name]
        except KeyError:
            raise KeyError(f"no tensor {name!r} in {self.path}") from None

    def close(self) -> None:
        if getattr(self, "_map", None) is not None:
            try:
                self._map.close()
            except BufferError:
                pass  # views are still alive: the mapping goes when the last one does
            self._map = None
        if getattr(self, "_file", None) is not None:
            self._file.close()
            self._file = None

    def __enter__(self) -> "GGUFFile":
        return self

    def __exit__(self, *exc) -> None:
        self.close()


def read(path: str | os.PathLike) -> GGUFFile:
    """Opens and parses a GGUF file (see :class:`GGUFFile`)."""
    return GGUFFile(path)
