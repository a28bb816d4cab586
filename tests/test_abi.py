"""The native library loads and exports every entry point that include/*.h
declares (no device work is started)."""
import ctypes
import re
from pathlib import Path

import pytest

from tinyinfer_amd._native import LIBRARY

ROOT = Path(__file__).resolve().parent.parent


def _declared():
    names = set()
    for header in (ROOT / "include").glob("*.h"):
        text = header.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names |= set(re.findall(r"\b(mpx?_\w+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    assert LIBRARY.exists(), "build the library first (__graft_entry__.build())"
    lib = ctypes.CDLL(str(LIBRARY))
    declared = _declared()
    assert len(declared) > 30
    missing = [n for n in declared if not hasattr(lib, n)]
    assert not missing, missing


def test_headers_are_plain_c():
    for header in (ROOT / "include").glob("*.h"):
        text = header.read_text()
        assert 'extern "C"' in text
        includes = re.findall(r"#include\s*[<\"]([^>\"]+)[>\"]", text)
        assert set(includes) <= {"stddef.h", "stdint.h"}, includes
