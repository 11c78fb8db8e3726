"""Dequantisation of table rows in their GGML wire form, on the device: the
drop-ins for the table formats of ``engraft/replica/dequant.py``
(``dequant_f32``, ``dequant_bf16``, ``dequant_q8_0``, ``dequant_iq4_nl``,
``:71-93, 127-147``).

``DeviceTable.read_rows_raw`` returns rows as GGML blocks (``[n, blocks *
block_bytes]`` uint8), so a caller that does
``dequant_q8_0(torch.from_numpy(raw).reshape(n, -1, 34))`` as it would with the
reference gets the same values here.  Each function keeps the reference's
signature and contract: a uint8 tensor whose last axis is one block
(``AssertionError`` otherwise), the result ``[..., values_per_block]`` in
``out_dtype`` on the input's device.  The decode runs in ``eg_dequant_blocks``
(one HIP launch); a CPU input is copied to the current GPU and the result
copied back.  Every decode is exact in fp32 (an 8-bit integer or a codebook
value times an fp16 scale, or a bit shift), so the values are bit-identical to
the reference's torch expressions.

The model-weight formats of the same module (Q6_K, IQ4_XS, IQ3_S) are not on
the table path and are not provided.
"""
from __future__ import annotations

import math

import torch

from . import _lib

# format -> (C format code, bytes per block, values per block)
_WIRE = {
    "F32": (_lib.FMT_CODES["f32"], 4, 1),
    "BF16": (_lib.FMT_CODES["bf16"], 2, 1),
    "Q8_0": (_lib.FMT_CODES["q8_0"], 34, 32),
    "IQ4_NL": (_lib.FMT_CODES["iq4_nl"], 18, 32),
}


def _dequant(name: str, data: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
    code, block_bytes, per_block = _WIRE[name]
    assert isinstance(data, torch.Tensor) and data.shape[-1] == block_bytes and data.dtype == torch.uint8
    lead = tuple(data.shape[:-1])
    n = math.prod(lead)
    dev = data.device if data.device.type == "cuda" else torch.device("cuda", torch.cuda.current_device())
    raw = data.to(dev).contiguous()
    out = torch.empty((n, per_block), dtype=torch.float32, device=dev)
    if n:
        _lib.call("eg_dequant_blocks", code, _lib.ptr(raw), n, _lib.ptr(out), _lib.stream_ptr(dev))
    return out.reshape(*lead, per_block).to(device=data.device, dtype=out_dtype)


def dequant_f32(data: torch.Tensor, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """``[..., 4]`` uint8 -> ``[..., 1]`` (the bytes as f32)."""
    return _dequant("F32", data, out_dtype)


def dequant_bf16(data: torch.Tensor, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """``[..., 2]`` uint8 -> ``[..., 1]``: the bf16 bits shifted into f32's top half."""
    return _dequant("BF16", data, out_dtype)


def dequant_q8_0(data: torch.Tensor, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """``[..., 34]`` uint8 Q8_0 blocks (fp16 ``d``, 32 int8) -> ``[..., 32]``,
    ``y = f32(q) * f32(d)``."""
    return _dequant("Q8_0", data, out_dtype)


def dequant_iq4_nl(data: torch.Tensor, out_dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """``[..., 18]`` uint8 IQ4_NL blocks (fp16 ``d``, 16 nibble bytes: low
    nibbles are values 0-15, high nibbles 16-31) -> ``[..., 32]``,
    ``y = d * KVALUES_IQ4NL[nibble]``."""
    return _dequant("IQ4_NL", data, out_dtype)


DEQUANT_FNS = {
    "F32": dequant_f32,
    "BF16": dequant_bf16,
    "Q8_0": dequant_q8_0,
    "IQ4_NL": dequant_iq4_nl,
}
