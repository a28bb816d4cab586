"""Loads the in-tree native library. There is no fallback: every entry point
of this package runs the HIP/C++ code in tinyinfer_amd/lib, and importing
without it raises."""
from __future__ import annotations

import ctypes
from pathlib import Path

LIBRARY = Path(__file__).resolve().parent / "lib" / "libminiprefix_hip.so"

F32P = ctypes.POINTER(ctypes.c_float)
I32P = ctypes.POINTER(ctypes.c_int32)

_lib = None


class NativeLibraryMissing(RuntimeError):
    pass


def library() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIBRARY.exists():
        raise NativeLibraryMissing(
            f"{LIBRARY} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`")
    _lib = ctypes.CDLL(str(LIBRARY))
    return _lib
