"""The C-ABI library: it loads, and exports every entry point ``include/wiretorch_amd.h``
declares, with the structure layouts the binding assumes. No GPU needed (nothing is
launched)."""

import ctypes
import re
from pathlib import Path

import pytest

from wiretorch_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "wiretorch_amd.h"


def declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^(?:int|int64_t)\s+(wt_\w+)\s*\(", text, re.M)))


def test_header_and_binding_agree():
    assert declared() == sorted(_lib.SIGNATURES)


@pytest.mark.skipif(not _lib.LIBRARY.exists(), reason="library not built")
def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_lib.LIBRARY))
    for name in declared():
        assert hasattr(lib, name), name
    _lib.load()


def test_struct_layouts_match_header():
    text = HEADER.read_text()
    for struct, cls in (("wt_tables", _lib.Tables), ("wt_side", _lib.Side),
                        ("wt_geometry", _lib.Geometry), ("wt_run_io", _lib.RunIO),
                        ("wt_backward_io", _lib.BackwardIO)):
        body = re.search(r"typedef struct \{([^{}]*)\}\s*" + struct + ";", text).group(1)
        body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
        names = re.findall(r"(\w+)\s*(?=[,;])", body)
        assert names == [f[0] for f in cls._fields_], struct
