"""The C-ABI library loads and exports every function include/*.h declares."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

from continuous_depth_batching_amd import _lib

INCLUDE = Path(__file__).resolve().parent.parent / "include"
DECL = re.compile(r"^\s*(?:int|int64_t|int32_t|void|const char\s*\*)\s+(cdb_\w+)\s*\(", re.M)


def declared_functions() -> set[str]:
    names: set[str] = set()
    for header in INCLUDE.glob("*.h"):
        names.update(DECL.findall(header.read_text()))
    return names


def test_header_declares_entry_points() -> None:
    assert "cdb_paged_decode_attention" in declared_functions()


def test_library_exports_every_declared_symbol() -> None:
    handle = ctypes.CDLL(str(_lib.LIBRARY_PATH))
    missing = [name for name in sorted(declared_functions()) if not hasattr(handle, name)]
    assert not missing, f"declared but not exported: {missing}"


def test_binding_covers_every_declared_symbol() -> None:
    assert declared_functions() == set(_lib.SIGNATURES)
    lib = _lib.lib()
    for name in _lib.SIGNATURES:
        assert getattr(lib, name).argtypes is not None


def test_workspace_size_query_without_gpu() -> None:
    lib = _lib.lib()
    assert lib.cdb_paged_decode_workspace_bytes(4, 16, 128, 100, 16, 2) == 4 * 4 * 16 * 130 * 4
    assert lib.cdb_paged_decode_workspace_bytes(-1, 16, 128, 100, 16, 2) == -1
