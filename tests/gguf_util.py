"""Writes small GGUF files (format v3, little endian) for the table-loader
tests: a header, typed metadata and per-head IQ4_NL tensors, laid out byte by
byte from the published GGUF format (test infrastructure)."""
from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_CODES = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
          I64: "<q", F64: "<d"}


def _str(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v, itype: int | None = None) -> bytes:
    if vtype == STRING:
        return _str(v)
    if vtype == ARRAY:
        out = struct.pack("<IQ", itype, len(v))
        return out + b"".join(_value(itype, x) for x in v)
    return struct.pack(_CODES[vtype], v)


def write_gguf(path, kv: list[tuple], tensors: list[tuple[str, tuple, int, bytes]], alignment: int = 32) -> list[int]:
    """``kv``: (key, type, value[, item type]); ``tensors``: (name, dims, ggml
    type, raw bytes).  Returns each tensor's absolute data offset."""
    head = b"GGUF" + struct.pack("<IQQ", 3, len(tensors), len(kv))
    for item in kv:
        key, vtype, v = item[:3]
        itype = item[3] if len(item) > 3 else None
        head += _str(key) + struct.pack("<I", vtype) + _value(vtype, v, itype)
    rel = []
    off = 0
    for _, _, _, data in tensors:
        rel.append(off)
        off += (len(data) + alignment - 1) // alignment * alignment
    for (name, dims, gtype, _), o in zip(tensors, rel):
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", gtype, o)
    start = (len(head) + alignment - 1) // alignment * alignment
    body = bytearray(head + b"\0" * (start - len(head)))
    for (_, _, _, data), o in zip(tensors, rel):
        body += b"\0" * (start + o - len(body)) + data
    with open(path, "wb") as f:
        f.write(bytes(body))
    return [start + o for o in rel]


def ple_table_file(path, spec, raw_heads: list[np.ndarray], image_token_id: int = 151_655) -> list[int]:
    """A per-head PLE table GGUF with ``spec``'s hash parameters and head h's
    raw IQ4_NL rows ``raw_heads[h]`` (uint8 ``[p_h, 90]``)."""
    kv = [("general.architecture", STRING, "qwen4exp"),
          ("general.alignment", U32, 32),
          ("qwen4exp.ple.eos_token_id", U32, spec.eos_token_id),
          ("qwen4exp.ple.image_token_id", U32, image_token_id),
          ("qwen4exp.ple.ngram_size", U32, spec.ngram_size),
          ("qwen4exp.ple.heads_per_ngram", U32, spec.heads_per_ngram),
          ("qwen4exp.ple.layer_multipliers", ARRAY, list(spec.layer_multipliers), U64),
          ("qwen4exp.ple.head_vocab_sizes", ARRAY, list(spec.head_vocab_sizes), U32),
          ("qwen4exp.ple.head_offsets", ARRAY, list(spec.head_offsets), U64)]
    tensors = [(f"ple_ngram_embd.{h}.weight", (160, int(r.shape[0])), 20, np.ascontiguousarray(r).tobytes())
               for h, r in enumerate(raw_heads)]
    return write_gguf(path, kv, tensors)
