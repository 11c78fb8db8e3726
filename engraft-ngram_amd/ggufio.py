"""A minimal GGUF reader for the PLE table file (host side).

The reference opens its table with the ``gguf`` package's ``GGUFReader``
(``engraft/table.py:50-88``), which is not available here; this module reads
the same file layout from the published GGUF format (v2/v3, little endian):

    magic b"GGUF", u32 version, u64 n_tensors, u64 n_kv
    n_kv x (string key, u32 value type, value)
    n_tensors x (string name, u32 n_dims, u64 dims[n_dims], u32 ggml type, u64 offset)
    padding to general.alignment (default 32), then the tensor data

with ``string = u64 length + UTF-8 bytes`` and array values ``u32 item type +
u64 count + items``.  ``read_gguf`` parses the metadata only (tensor data stays
in the file, read by offset); ``read_tensor_f32`` reads one F32 / F16 / Q8_0
tensor, ``read_rms_eps`` the RMS-norm epsilon of a (split) model file.
"""
from __future__ import annotations

import dataclasses
import re
import struct
from pathlib import Path

import numpy as np

GGUF_MAGIC = b"GGUF"
GGML_TYPE_IQ4_NL = 20

# value types: (struct code, size)
_SCALARS = {0: ("<B", 1), 1: ("<b", 1), 2: ("<H", 2), 3: ("<h", 2), 4: ("<I", 4), 5: ("<i", 4), 6: ("<f", 4),
            7: ("<?", 1), 10: ("<Q", 8), 11: ("<q", 8), 12: ("<d", 8)}
_STRING, _ARRAY = 8, 9


@dataclasses.dataclass(frozen=True)
class TensorInfo:
    name: str
    shape: tuple[int, ...]  # ne0 first (ne0 = values per row)
    ggml_type: int
    data_offset: int        # absolute offset in the file


class _Cursor:
    def __init__(self, f):
        self.f = f

    def read(self, n: int) -> bytes:
        b = self.f.read(n)
        if len(b) != n:
            raise ValueError("GGUF: unexpected end of file")
        return b

    def scalar(self, code: str, size: int):
        return struct.unpack(code, self.read(size))[0]

    def string(self) -> str:
        n = self.scalar("<Q", 8)
        return self.read(n).decode("utf-8")

    def value(self, vtype: int):
        if vtype in _SCALARS:
            return self.scalar(*_SCALARS[vtype])
        if vtype == _STRING:
            return self.string()
        if vtype == _ARRAY:
            itype = self.scalar("<I", 4)
            count = self.scalar("<Q", 8)
            return [self.value(itype) for _ in range(count)]
        raise ValueError(f"GGUF: unknown value type {vtype}")


@dataclasses.dataclass
class GGUFFile:
    path: Path
    version: int
    fields: dict
    tensors: dict[str, TensorInfo]
    alignment: int


def read_gguf(path: str | Path) -> GGUFFile:
    """The metadata and tensor directory of a GGUF file."""
    path = Path(path)
    with open(path, "rb") as f:
        c = _Cursor(f)
        if c.read(4) != GGUF_MAGIC:
            raise ValueError(f"{path}: not a GGUF file")
        version = c.scalar("<I", 4)
        if version not in (2, 3):
            raise ValueError(f"{path}: GGUF version {version} (2 and 3 are read)")
        n_tensors = c.scalar("<Q", 8)
        n_kv = c.scalar("<Q", 8)
        fields = {}
        for _ in range(n_kv):
            key = c.string()
            fields[key] = c.value(c.scalar("<I", 4))
        infos = []
        for _ in range(n_tensors):
            name = c.string()
            n_dims = c.scalar("<I", 4)
            dims = tuple(c.scalar("<Q", 8) for _ in range(n_dims))
            gtype = c.scalar("<I", 4)
            off = c.scalar("<Q", 8)
            infos.append((name, dims, gtype, off))
        alignment = int(fields.get("general.alignment", 32))
        pos = f.tell()
        data_start = (pos + alignment - 1) // alignment * alignment
    tensors = {n: TensorInfo(n, d, t, data_start + o) for n, d, t, o in infos}
    return GGUFFile(path, version, fields, tensors, alignment)


# ggml tensor types read by read_tensor_f32: (block values, block bytes)
GGML_TYPE_F32 = 0
GGML_TYPE_F16 = 1
GGML_TYPE_Q8_0 = 8
_BLOCKS = {GGML_TYPE_F32: (1, 4), GGML_TYPE_F16: (1, 2), GGML_TYPE_Q8_0: (32, 34)}


def read_tensor_f32(gf: GGUFFile, name: str, expected_type: int | None = None) -> np.ndarray:
    """Tensor ``name`` as f32 numpy, shaped with ne0 last (``[ne1, ne0]`` for a
    matrix).  F32, F16 and Q8_0 (blocks of an fp16 scale d and 32 int8 q,
    value d*q) are read.  ``expected_type``: raise ValueError on another type
    (``engraft/lens.py:236-244``)."""
    if name not in gf.tensors:
        raise KeyError(f"{name}: tensor missing in {gf.path}")
    info = gf.tensors[name]
    if expected_type is not None and info.ggml_type != expected_type:
        raise ValueError(f"{name}: expected ggml type {expected_type}, got {info.ggml_type}")
    if info.ggml_type not in _BLOCKS:
        raise ValueError(f"{name}: ggml type {info.ggml_type} is not read (F32, F16, Q8_0)")
    n = 1
    for d in info.shape:
        n *= int(d)
    per, nbytes = _BLOCKS[info.ggml_type]
    if n % per:
        raise ValueError(f"{name}: {n} values are not whole blocks of {per}")
    raw = np.fromfile(gf.path, dtype=np.uint8, count=n // per * nbytes, offset=info.data_offset)
    if raw.size != n // per * nbytes:
        raise ValueError(f"{name}: tensor data past the end of {gf.path}")
    if info.ggml_type == GGML_TYPE_F32:
        vals = raw.view("<f4").astype(np.float32)
    elif info.ggml_type == GGML_TYPE_F16:
        vals = raw.view("<f2").astype(np.float32)
    else:
        blocks = raw.reshape(-1, 34)
        d = blocks[:, :2].copy().view("<f2").astype(np.float32)  # [n_blocks, 1]
        q = blocks[:, 2:].view(np.int8).astype(np.float32)
        vals = (q * d).reshape(-1)
    return vals.reshape(tuple(int(x) for x in reversed(info.shape)))


def read_rms_eps(path: str | Path) -> float:
    """``qwen4exp.attention.layer_norm_rms_epsilon`` of a model file; for a
    split file (``…-NNNNN-of-MMMMM.gguf``) it is read from shard 1, which alone
    holds the model metadata (``engraft/lens.py:490-518``)."""
    path = Path(path)
    m = re.search(r"(\d{5})-of-(\d{5})", path.name)
    src = path
    if m is not None:
        src = path.with_name(path.name[:m.start(1)] + "00001" + path.name[m.end(1):])
        if not src.exists():
            raise FileNotFoundError(f"eps not given explicitly and shard 1 not found: {src}")
    key = "qwen4exp.attention.layer_norm_rms_epsilon"
    fields = read_gguf(src).fields
    if key not in fields:
        raise KeyError(f"{key}: missing in {src}")
    return float(fields[key])
