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


def q8_0_blocks(x: np.ndarray) -> tuple[bytes, np.ndarray]:
    """GGML Q8_0 bytes of ``x`` (blocks of 32 along the last axis: fp16 d, then
    32 int8 q) and their value d*q, the closed form a reader must give."""
    from oracle import formats as F
    x = np.ascontiguousarray(x, dtype=np.float32)
    flat = x.reshape(-1, 32)
    q, d16 = F.quant_q8_0(flat.reshape(-1, 32))  # one block per row
    raw = np.concatenate([d16.reshape(-1, 1).view(np.uint8), q.view(np.uint8)], axis=1)  # [n_blocks, 34]
    vals = (q.astype(np.float32) * d16.astype(np.float32)).reshape(x.shape)
    return raw.tobytes(), vals


def ple_model_files(dir_path, w: dict, eps: float, layer: int = 1, split: bool = True):
    """A model GGUF holding ``blk.<layer>.ple_*`` (key/value Q8_0, the rest F32)
    -- as shard 2 of a 2-shard split whose shard 1 holds the metadata, or one
    file with both.  Returns (path to pass, dequantised weights dict)."""
    from pathlib import Path
    dir_path = Path(dir_path)
    kb, kv_vals = q8_0_blocks(w["w_key"])
    vb, vv_vals = q8_0_blocks(w["w_value"])
    f32 = lambda a: np.ascontiguousarray(a, dtype=np.float32)
    dims = lambda a: tuple(reversed(np.asarray(a).shape))  # ne0 first
    tensors = [(f"blk.{layer}.ple_key.weight", dims(w["w_key"]), 8, kb),
               (f"blk.{layer}.ple_value.weight", dims(w["w_value"]), 8, vb)]
    for name in ("norm_key", "norm_query", "norm_conv", "conv1d"):
        tensors.append((f"blk.{layer}.ple_{name}.weight", dims(w[name]), 0, f32(w[name]).tobytes()))
    meta = [("general.architecture", STRING, "qwen4exp"),
            ("qwen4exp.attention.layer_norm_rms_epsilon", F32, float(eps))]
    if split:
        write_gguf(dir_path / "m-00001-of-00002.gguf", meta + [("split.count", U16, 2)], [])
        path = dir_path / "m-00002-of-00002.gguf"
        write_gguf(path, [("split.count", U16, 2)], tensors)
    else:
        path = dir_path / "m.gguf"
        write_gguf(path, meta, tensors)
    vals = dict(w)
    vals["w_key"], vals["w_value"] = kv_vals, vv_vals
    return path, vals
