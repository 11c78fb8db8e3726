"""ctypes binding of the C ABI declared in ``include/engraft_ngram.h``.

The library is loaded on first use and never replaced by anything else: if
``libengraft_ngram.so`` is missing or does not load, every product entry point
raises ``RuntimeError`` (there is no CPU fallback).
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_int32, c_int64, c_uint64, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libengraft_ngram.so"
# the C++ autograd functions over the library's entry points (csrc/eg_autograd.cpp)
EXT_NAME = "_eg_autograd"
EXT_PATH = Path(__file__).resolve().parent / "_eg_autograd.so"

EG_MAX_NGRAM = 4
EG_MAX_HEADS = 32
EG_MAX_LAYERS = 2

EG_OK = 0
EG_ERR_ARG = -1
EG_ERR_HIP = -2
EG_ERR_UNSUPPORTED = -3
EG_ERR_WORKSPACE = -4

FMT_BF16 = 1
FMT_Q8_0 = 2
FMT_MXFP8 = 3
FMT_IQ4_NL = 4
FMT_F32 = 5

ABI_VERSION = 4  # EG_ABI_VERSION of include/engraft_ngram.h these structures follow

FMT_CODES = {"bf16": FMT_BF16, "q8_0": FMT_Q8_0, "mxfp8": FMT_MXFP8, "iq4_nl": FMT_IQ4_NL, "f32": FMT_F32}


class EgHashSpec(ctypes.Structure):
    _fields_ = [
        ("eos_token_id", c_uint64),
        ("ngram_size", c_int32),
        ("heads_per_ngram", c_int32),
        ("layer_multipliers", c_uint64 * EG_MAX_NGRAM),
        ("head_multipliers", c_void_p),
        ("head_vocab_sizes", c_uint64 * EG_MAX_HEADS),
        ("head_offsets", c_int64 * EG_MAX_HEADS),
    ]


class EgTable(ctypes.Structure):
    _fields_ = [
        ("fmt", c_int32),
        ("dim", c_int32),
        ("n_rows", c_int64),
        ("payload", c_void_p),
        ("scales", c_void_p),
        ("row_stride", c_int64),
    ]


class EgOverlay(ctypes.Structure):
    _fields_ = [
        ("n", c_int64),
        ("ids", c_void_p),
        ("index", c_void_p),
        ("rows", EgTable),
        ("bitmap", c_void_p),
        ("n_bits", c_int64),
    ]


class EgAdam(ctypes.Structure):
    _fields_ = [
        ("lr", ctypes.c_double),
        ("beta1", ctypes.c_double),
        ("beta2", ctypes.c_double),
        ("eps", ctypes.c_double),
        ("step", c_int64),
        ("dense", c_int32),
        ("l2_coef", ctypes.c_float),
        ("anchor", c_void_p),
    ]


class EgDescentState(ctypes.Structure):
    _fields_ = [
        ("n", c_int64),
        ("dim", c_int32),
        ("ids", c_void_p),
        ("master", c_void_p),
        ("m", c_void_p),
        ("v", c_void_p),
        ("stamp", c_void_p),
        ("quant", EgTable),
        ("index", c_void_p),
        ("index_capacity", c_int64),
        ("row_stride", c_int64),
    ]


class EgGemmOperands(ctypes.Structure):
    _fields_ = [
        ("a_hi", c_void_p),
        ("a_lo", c_void_p),
        ("lda", c_int64),
        ("b_hi", c_void_p),
        ("b_lo", c_void_p),
        ("ldb", c_int64),
        ("b2_hi", c_void_p),
        ("b2_lo", c_void_p),
        ("ldb2", c_int64),
        ("k", c_int64),
    ]


class EgGemmF32Operands(ctypes.Structure):
    _fields_ = [
        ("a", c_void_p),
        ("lda", c_int64),
        ("b", c_void_p),
        ("ldb", c_int64),
        ("b2", c_void_p),
        ("ldb2", c_int64),
        ("k", c_int64),
    ]


# name -> (restype, argtypes); every symbol the header declares.
SIGNATURES = {
    "eg_last_error": (c_char_p, []),
    "eg_abi_version": (c_int32, []),
    "eg_hash_rows": (c_int32, [POINTER(EgHashSpec), c_void_p, c_int64, c_int64, c_void_p, c_int32, c_void_p,
                               c_void_p]),
    "eg_forward": (c_int32, [c_int32, POINTER(EgHashSpec), POINTER(EgTable), POINTER(EgOverlay), c_void_p,
                             c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "eg_forward_slots": (c_int32, [c_int32, POINTER(EgHashSpec), POINTER(EgTable), POINTER(EgOverlay), c_void_p,
                                   c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "eg_forward_rows": (c_int32, [c_int32, POINTER(EgTable), POINTER(EgOverlay), c_void_p, c_int64, c_int32,
                                  c_void_p, c_void_p, c_void_p]),
    "eg_stream_copy": (c_int32, [c_void_p, c_void_p, c_int64, c_void_p]),
    "eg_dequant_blocks": (c_int32, [c_int32, c_void_p, c_int64, c_void_p, c_void_p]),
    "eg_ple_gate": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int32,
                              c_int32, ctypes.c_float, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "eg_ple_conv_backward": (c_int32, [c_void_p, c_int64, c_int64, c_int32, c_int32, c_void_p, c_int32, c_int32,
                                       c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p]),
    "eg_ple_gate_backward": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_int32, c_int32,
                                       c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "eg_ple_gate_backward_planes": (c_int32, [c_void_p] * 11 + [c_int64, c_int32, c_int32, c_int32, c_int32] +
                                    [c_void_p] * 7),
    "eg_ple_weight_grads_workspace_size": (ctypes.c_size_t, [c_int64, c_int32, c_int32, c_int32]),
    "eg_ple_weight_grads": (c_int32, [c_void_p] * 11 + [c_int64, c_void_p, c_int64, c_int32, c_int32, c_int32,
                                                        c_int32] + [c_void_p] * 5 + [ctypes.c_size_t, c_void_p]),
    "eg_ple_conv": (c_int32, [c_void_p, c_int64, c_int64, c_int32, c_int32, c_void_p, c_int32, c_int32, c_int32,
                              c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "eg_ple_rms": (c_int32, [c_void_p, c_int64, c_int32, c_int32, c_void_p, ctypes.c_float, c_void_p, c_void_p]),
    "eg_split_bf16": (c_int32, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p]),
    "eg_gemm_workspace_size": (c_int64, [c_int64, c_int64, c_int64, c_int64, c_int32]),
    "eg_gemm_f32_workspace_size": (c_int64, [c_int64, c_int64, c_int64, c_int64, c_int32]),
    "eg_gemm_bf16x3": (c_int32, [POINTER(EgGemmOperands), c_int32, c_int64, c_int64, c_int64, c_void_p, c_int64,
                                 c_void_p, c_int64, c_int32, c_int32, c_void_p, c_int64, c_void_p]),
    "eg_gemm_f32": (c_int32, [POINTER(EgGemmF32Operands), c_int32, c_int64, c_int64, c_int64, c_void_p, c_int64,
                              c_void_p, c_int64, c_int32, c_int32, c_void_p, c_int64, c_void_p]),
    "eg_split_bf16x6": (c_int32, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p]),
    "eg_gemm_bf16x6": (c_int32, [POINTER(EgGemmOperands), POINTER(EgGemmOperands), c_int32, c_int64, c_int64,
                                 c_int64, c_void_p, c_int64, c_void_p, c_int64, c_int32, c_int32, c_void_p, c_int64,
                                 c_void_p]),
    "eg_forward_decode": (c_int32, [c_int32, POINTER(EgHashSpec), POINTER(EgTable), POINTER(EgOverlay), c_void_p,
                                    c_int64, c_int32, c_void_p, c_void_p, c_void_p, c_void_p]),
    "eg_forward_timed": (c_int32, [c_int32, POINTER(EgHashSpec), POINTER(EgTable), POINTER(EgOverlay), c_void_p,
                                   c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                   c_void_p]),
    "eg_gather": (c_int32, [POINTER(EgTable), POINTER(EgOverlay), c_void_p, c_int64, c_int32, c_void_p,
                            c_void_p]),
    "eg_synth_table": (c_int32, [POINTER(EgTable), c_uint64, c_void_p, c_int64, c_int64, c_void_p]),
    "eg_backward_workspace_size": (ctypes.c_size_t, [c_int64, c_int64]),
    "eg_build_row_index": (c_int32, [c_void_p, c_int64, c_void_p, c_int64, c_void_p]),
    "eg_lookup_rows": (c_int32, [c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_void_p]),
    "eg_gather_slots": (c_int32, [POINTER(EgTable), c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_int64,
                                  c_void_p, c_void_p]),
    "eg_scatter_grad_slots": (c_int32, [c_void_p, c_int32, c_void_p, c_int64, c_int32, c_int32, c_int64, c_void_p,
                                        c_void_p, ctypes.c_size_t, c_void_p]),
    "eg_scatter_grad_plan_slots": (c_int32, [c_void_p, c_int64, c_int32, c_int64, c_void_p, ctypes.c_size_t,
                                             c_void_p]),
    "eg_scatter_grad_apply": (c_int32, [c_void_p, c_int32, c_int64, c_int32, c_int32, c_int64, c_void_p, c_int32,
                                        c_void_p, ctypes.c_size_t, c_void_p]),
    "eg_scatter_grad": (c_int32, [c_void_p, c_int32, c_void_p, c_int64, c_int32, c_int32, c_void_p, c_int64,
                                  c_void_p, c_void_p, ctypes.c_size_t, c_void_p]),
    "eg_descent_step": (c_int32, [c_void_p, c_int32, c_void_p, c_int64, c_int32, POINTER(EgDescentState),
                                  POINTER(EgAdam), POINTER(EgTable), c_void_p, ctypes.c_size_t, c_void_p]),
    "eg_descent_plan_slots": (c_int32, [c_void_p, c_int64, c_int32, POINTER(EgDescentState), c_void_p,
                                        ctypes.c_size_t, c_void_p]),
    "eg_descent_plan": (c_int32, [c_void_p, c_int64, c_int32, POINTER(EgDescentState), c_void_p, ctypes.c_size_t,
                                  c_void_p]),
    "eg_descent_apply": (c_int32, [c_void_p, c_int32, c_int64, c_int32, POINTER(EgDescentState), POINTER(EgAdam),
                                   POINTER(EgTable), c_void_p, ctypes.c_size_t, c_void_p]),
    "eg_descent_step_noalloc": (c_int32, [c_void_p, c_int32, c_void_p, c_int64, c_int32, POINTER(EgDescentState),
                                          POINTER(EgAdam), POINTER(EgTable), c_void_p]),
    "eg_descent_step_noalloc_max_bytes": (ctypes.c_size_t, []),
    "eg_quantize_rows": (c_int32, [c_void_p, c_int64, c_int32, c_void_p, POINTER(EgTable), c_void_p]),
    "eg_scan_overlay": (c_int32, [POINTER(EgHashSpec), c_void_p, c_int32, c_int64, c_int64, c_void_p, c_int64,
                                  c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "eg_build_id_bitmap": (c_int32, [c_void_p, c_int64, c_void_p, c_int64, c_void_p]),
    "eg_id_bitmap_words": (c_int64, [c_int64]),
}

_LIB = None


def load(path: Path | None = None) -> ctypes.CDLL:
    """Loads (once) and returns the library; raises RuntimeError if absent."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise RuntimeError(
            f"HIP library {p} not found: build it with `python engraft-ngram_amd/build.py` "
            "(or __graft_entry__.build()); there is no CPU fallback")
    lib = ctypes.CDLL(str(p))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name, None)
        if fn is None:
            if path is None:
                raise RuntimeError(f"HIP library {p} lacks {name}: rebuild it with `python engraft-ngram_amd/build.py`")
            continue  # another build of the library, loaded by path: only what it has
        fn.restype = restype
        fn.argtypes = argtypes
    if lib.eg_abi_version() != ABI_VERSION:
        raise RuntimeError(f"HIP library {p} has ABI version {lib.eg_abi_version()}, this package needs "
                           f"{ABI_VERSION}: rebuild it with `python engraft-ngram_amd/build.py`")
    if path is None:
        _LIB = lib
    return lib


_EXT = None


def autograd_ext():
    """The C++ autograd module (``_eg_autograd.so``, built beside the library
    by the same build), bound once to the loaded library's entry points;
    raises RuntimeError if it is absent (no Python stand-in)."""
    global _EXT
    if _EXT is not None:
        return _EXT
    if not EXT_PATH.exists():
        raise RuntimeError(f"{EXT_PATH} not found: build it with `python engraft-ngram_amd/build.py` "
                           "(or __graft_entry__.build())")
    import importlib.machinery
    import importlib.util

    import torch  # noqa: F401  (the module links torch's libraries)

    loader = importlib.machinery.ExtensionFileLoader(EXT_NAME, str(EXT_PATH))
    spec = importlib.util.spec_from_file_location(EXT_NAME, str(EXT_PATH), loader=loader)
    mod = importlib.util.module_from_spec(spec)
    loader.exec_module(mod)
    lib = load()
    mod.init(*(ctypes.cast(getattr(lib, f), c_void_p).value
               for f in ("eg_gather_slots", "eg_scatter_grad_apply", "eg_last_error")))
    _EXT = mod
    return mod


class EgError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"engraft_ngram error {code}: {message}")
        self.code = code


def check(code: int) -> None:
    if code != EG_OK:
        msg = load().eg_last_error()
        msg = msg.decode() if msg else ""
        if code == EG_ERR_ARG:
            raise ValueError(msg)
        raise EgError(code, msg)


def call(name: str, *args) -> None:
    check(getattr(load(), name)(*args))


def stream_ptr(device=None) -> int:
    """The current HIP stream of ``device`` (default: the current device) as
    an integer.  torch's raw-stream query when it has one (a few hundred ns,
    against ~2 us for building the ``torch.cuda.Stream`` object)."""
    import torch

    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is None:
        return int(torch.cuda.current_stream(device).cuda_stream)
    if isinstance(device, torch.device):
        idx = device.index
    elif device is None or isinstance(device, int):
        idx = device
    else:
        idx = torch.device(device).index
    return int(raw(torch.cuda.current_device() if idx is None else idx))


def ptr(t) -> int | None:
    """Device pointer of a tensor (None for None)."""
    if t is None:
        return None
    return int(t.data_ptr())
