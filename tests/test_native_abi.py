"""The C-ABI library loads and exports every symbol include/fast_mimi_amd.h
declares (no kernel is launched here: this suite runs without a GPU)."""

from __future__ import annotations

import re
import subprocess

import pytest

from conftest import REPO
from fast_mimi_amd import _native as nat

HEADER = REPO / "include" / "fast_mimi_amd.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t)\s+(fm_\w+)\s*\(", text, re.M)))


def test_header_declares_the_bound_entry_points():
    assert declared_symbols() == sorted(nat.exported_symbols())


def test_library_exports_every_declared_symbol():
    if not nat.LIBRARY_PATH.is_file():
        pytest.skip("library not built")
    lib = nat.library()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(nat.LIBRARY_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (fm_\w+)", out))
    assert set(declared_symbols()) <= exported
    assert lib.fm_abi_version() == nat.ABI_VERSION


def test_workspace_query_is_host_only():
    if not nat.LIBRARY_PATH.is_file():
        pytest.skip("library not built")
    lib = nat.library()
    a = lib.fm_rvq_workspace_bytes(125, 256, 2048)
    b = lib.fm_rvq_workspace_bytes(250, 256, 2048)
    assert 0 < a < b


def test_status_codes_map_to_errors():
    with pytest.raises(nat.NativeError, match="bad argument"):
        nat.check(1000, "fm_x")
    with pytest.raises(nat.NativeError, match="hipError_t 700"):
        nat.check(700, "fm_x")
    nat.check(0, "fm_x")
