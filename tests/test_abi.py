"""The C-ABI library loads and exports every symbol include/engraft_ngram.h
declares (no compute call: this runs without a GPU)."""
from __future__ import annotations

import ctypes
import re

import pytest

from tests.conftest import ROOT

HEADER = ROOT / "include" / "engraft_ngram.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(eg_[a-z_0-9]+)\s*\(", text, flags=re.M)))


def test_header_declares_entry_points():
    names = declared_symbols()
    for must in ("eg_last_error", "eg_hash_rows", "eg_forward", "eg_gather"):
        assert must in names


def test_library_exports_every_declared_symbol():
    from engraft_ngram_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.fail(f"{_lib.LIB_PATH} not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert not missing, f"declared in {HEADER.name} but not exported: {missing}"
    # every declared symbol has a ctypes signature in the binding
    assert set(declared_symbols()) <= set(_lib.SIGNATURES)


def test_abi_version_and_error_string():
    from engraft_ngram_amd import _lib

    lib = _lib.load()
    assert lib.eg_abi_version() == 1
    # an argument error is reported without touching the device
    spec = _lib.EgHashSpec()
    spec.ngram_size = 9
    rc = lib.eg_hash_rows(ctypes.byref(spec), None, 0, 0, None, 1, None, None)
    assert rc == _lib.EG_ERR_ARG
    assert b"ngram_size" in lib.eg_last_error()
