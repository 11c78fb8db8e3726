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


def test_autograd_module_loads_and_checks_its_arguments():
    """The C++ autograd module (OverlayEmb's gather) is built beside the
    library, binds to the library's entry points, and refuses a malformed plan
    on the host before calling them."""
    import torch

    from engraft_ngram_amd import _lib

    if not _lib.EXT_PATH.exists():
        pytest.fail(f"{_lib.EXT_PATH} not built: run __graft_entry__.build()")
    ext = _lib.autograd_ext()
    assert callable(ext.init) and callable(ext.gather_slots)
    rows = torch.zeros((3, 16), dtype=torch.int32)
    ws = torch.empty(0, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="slot_var"):
        ext.gather_slots(torch.zeros((2, 128)), rows, rows[:2].clone(), ws, 0, 128, 0)
    with pytest.raises(RuntimeError, match="rows_var"):
        ext.gather_slots(torch.zeros((2, 64)), rows, rows.clone(), ws, 0, 128, 0)
    with pytest.raises(RuntimeError, match="ws"):
        ext.gather_slots(torch.zeros((2, 128)), rows, rows.clone(), torch.empty(0), 0, 128, 0)


def test_abi_version_and_error_string():
    from engraft_ngram_amd import _lib

    lib = _lib.load()
    assert lib.eg_abi_version() == 4
    # an argument error is reported without touching the device
    spec = _lib.EgHashSpec()
    spec.ngram_size = 9
    rc = lib.eg_hash_rows(ctypes.byref(spec), None, 0, 0, None, 1, None, None)
    assert rc == _lib.EG_ERR_ARG
    assert b"ngram_size" in lib.eg_last_error()


def _rejects(fn, *args) -> tuple[int, str]:
    from engraft_ngram_amd import _lib
    rc = fn(*args)
    return rc, (_lib.load().eg_last_error() or b"").decode()


def test_host_side_argument_checks():
    """Every entry point rejects a bad argument on the host, before any launch,
    with a status and a message (the Python layer raises ValueError for
    EG_ERR_ARG, as the reference raises for bad shapes); these run without a GPU."""
    from engraft_ngram_amd import _lib
    lib = _lib.load()
    spec = _lib.EgHashSpec()
    spec.ngram_size, spec.heads_per_ngram = 3, 8
    tab = _lib.EgTable()
    tab.fmt, tab.dim, tab.n_rows = _lib.FMT_BF16, 128, 10
    cases = [
        ("n_layers", _lib.EG_ERR_ARG, lib.eg_forward, 3, ctypes.byref(spec), ctypes.byref(tab), None, None, 1, 0, None,
         None, None, None, None),
        ("NULL", _lib.EG_ERR_ARG, lib.eg_gather, None, None, None, 1, 1, None, None),
        ("NULL", _lib.EG_ERR_ARG, lib.eg_descent_step, None, 0, None, 1, 16, None, None, None, None, 0, None),
        ("Q8_0 or MXFP8", _lib.EG_ERR_ARG, lib.eg_quantize_rows, None, 1, 128, None, ctypes.byref(tab), None),
        ("n_embd", _lib.EG_ERR_ARG, lib.eg_ple_gate, None, None, None, None, None, None, 1, 4, 5000, 1e-6, None,
         None, None, None, None),
        ("taps", _lib.EG_ERR_ARG, lib.eg_ple_conv, None, 0, 1, 4, 64, None, 9, 3, 0, None, None, None, None, None,
         None),
        ("dilation", _lib.EG_ERR_UNSUPPORTED, lib.eg_ple_conv_backward, None, 0, 1, 4, 64, None, 4, 11, None, None,
         None, 0, None, None),
        ("hc=5", _lib.EG_ERR_UNSUPPORTED, lib.eg_ple_gate_backward, *([None] * 11), 1, 5, 64, 0, 0, None, None,
         None, None, None),
        ("taps", _lib.EG_ERR_UNSUPPORTED, lib.eg_ple_weight_grads, *([None] * 11), 0, None, 4, 4, 64, 9, 3,
         None, None, None, None, None, 0, None),
        ("at least one position", _lib.EG_ERR_ARG, lib.eg_ple_weight_grads, *([None] * 11), 0, None, 0, 4, 64, 4,
         3, None, None, None, None, None, 0, None),
        ("taps", _lib.EG_ERR_ARG, lib.eg_ple_conv_backward, None, 0, 1, 4, 64, None, 9, 1, None, None, None, 0,
         None, None),
    ]
    # bf16x6: the third plane, and the two plane sets' K segments checked against each other
    hm, hl = (_lib.EgGemmOperands * 2)(), (_lib.EgGemmOperands * 2)()
    for o, k in ((hm[0], 32), (hl[0], 64)):
        o.a_hi = o.a_lo = o.b_hi = o.b_lo = 256
        o.lda = o.ldb = 64
        o.k = k
    cases += [
        ("NULL", _lib.EG_ERR_ARG, lib.eg_split_bf16x6, ctypes.c_void_p(256), 4, 32, 32, ctypes.c_void_p(256),
         ctypes.c_void_p(256), None, None),
        ("n_seg", _lib.EG_ERR_ARG, lib.eg_gemm_bf16x6, hm, hl, 3, 8, 8, 0, None, 8, None, 0, 0, 0, None, 0, None),
        ("same K segments", _lib.EG_ERR_ARG, lib.eg_gemm_bf16x6, hm, hl, 1, 8, 8, 0, ctypes.c_void_p(256), 8, None,
         0, 0, 0, None, 0, None),
    ]
    for needle, code, fn, *args in cases:
        rc, msg = _rejects(fn, *args)
        assert rc == code, (fn.__name__, rc, msg)
        assert needle in msg, (fn.__name__, msg)
    # the workspace check: too small a workspace is its own status
    need = lib.eg_backward_workspace_size(1000, 100)
    assert need > 0 and lib.eg_backward_workspace_size(2000, 100) > need
    ids = ctypes.c_int32(0)
    rc, msg = _rejects(lib.eg_scatter_grad, ctypes.c_void_p(8), 0, ctypes.c_void_p(8), 10, 16, 128,
                       ctypes.byref(ids), 1, ctypes.c_void_p(8), ctypes.c_void_p(8), 16, None)
    assert rc == _lib.EG_ERR_WORKSPACE and "workspace" in msg
    with pytest.raises(ValueError):
        _lib.check(_lib.EG_ERR_ARG)
