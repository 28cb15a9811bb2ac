"""The C-ABI library loads and exports every symbol include/exl3_mi355x.h declares.

No compute calls: this runs without a GPU."""

import ctypes
import pathlib
import re

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "exl3_mi355x.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(exl3_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_functions()
    assert "exl3_dequant_trellis" in names and "exl3_last_error" in names


def test_library_exports_every_declared_symbol():
    from vllm_exl3_amd import _lib

    lib = _lib.load()
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # and the Python binding types every declared function
    assert set(declared_functions()) <= set(_lib.exported_symbols())


def test_abi_version_and_error_plumbing():
    from vllm_exl3_amd import _lib

    lib = _lib.load()
    assert lib.exl3_abi_version() == 4
    # a validation failure is reported before any launch (no GPU needed)
    status = lib.exl3_dequant_trellis(None, 8, 8, 5, 1, None, None, None, None)
    assert status == -1
    assert "K must be one of" in _lib.last_error()


def test_module_attributes_match_reference():
    from vllm_exl3_amd import vllm_exl3_c as m

    assert m.P2B_MOE_ABI_VERSION == 4 and m.P2B_MOE_MIXED_K and m.P2B_MOE_PADDED
