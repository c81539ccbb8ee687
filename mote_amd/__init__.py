"""MI355X (gfx950) implementation of Mote's Q4_0 quantized-linear hot path.

The compute lives in ``libmote_hip.so`` (hand-written HIP kernels behind the C
ABI of ``include/mote_hip.h``); this package binds it with ctypes.  There is no
CPU fallback: calling into the package without the built library raises
:class:`mote_amd._ffi.LibraryNotBuilt`.
"""

from ._ffi import HipError, LibraryNotBuilt, LIBRARY, lib  # noqa: F401

__all__ = ["HipError", "LibraryNotBuilt", "LIBRARY", "lib"]
