"""Oracle: table row formats (TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py).

Row formats, all ``D`` values per row in blocks of 32:

* ``bf16``  -- ``[rows, D]`` bfloat16 (config 0).  Dequant = ``bits << 16``
  (``engraft/replica/dequant.py:77-83``).
* ``q8_0``  -- GGML Q8_0 semantics in a *split* layout: int8 payload
  ``[rows, D]`` plus one fp16 scale per 32 values ``[rows, D/32]`` (configs 1-3).
  Dequant ``y = f32(int8) * f32(fp16 d)`` (``engraft/replica/dequant.py:86-93``).
* ``mxfp8`` -- OCP MX: e4m3 payload ``[rows, D]`` + one e8m0 scale per 32
  values ``[rows, D/32]`` (config 4; not in the reference, build-defined).
  Dequant ``y = f32(e4m3) * 2**(e - 127)``.
* ``iq4_nl`` -- the reference's real table format, interleaved 18-byte blocks
  (fp16 d, 16 nibble bytes), ``engraft/table.py:18-29, 147-169``.
* ``f32``   -- ``[rows, D]`` float32 (``.pleo`` overlays, ``engraft/lens.py:33-59``).

Every dequantisation here is exact in fp32 (<= 8-bit integer or 4-bit-mantissa
value times an fp16 or power-of-two scale), so any correct implementation is
bit-identical to these.

Requantisation (build-defined; the reference stores fp32 overlays and never
requantises, ``engraft/lens.py:33-46``):

* ``quant_q8_0``: per 32-block ``amax = max|x|``, ``d = fp16_rne(amax / 127)``
  (fp32 IEEE division), ``q = clamp(rint(x / f32(d)), -127, 127)`` (fp32 IEEE
  division, round half to even); ``d == 0`` gives ``q = 0``.
* ``quant_mxfp8``: per 32-block shared exponent ``e`` = the smallest integer
  with ``amax * 2**-e <= 448`` (``floor(log2 amax) - 8``, read from the fp32
  bits, plus one when that would saturate), clamped to [-127, 127]; elements
  ``e4m3_rne(clamp(x * 2**-e, -448, 448))``; ``amax == 0`` gives ``e = -127``
  and zero elements.  (OCP's ``floor(log2 amax) - emax`` would clip block
  maxima in [448, 512) * 2**e by up to 12.5 %.)

Pinning (tests/test_oracle_formats.py): closed forms against hand-built blocks,
the reference's synthetic ``row_is_zero`` vector (``tests/test_table.py:57-63``),
e4m3 decoding against torch's ``float8_e4m3fn`` (library routine) over all 256
codes, requantisation round-trip bounds and exhaustive small-block checks.
"""
from __future__ import annotations

import numpy as np

BLOCK = 32

# ggml-common.h kvalues_iq4nl as restated in engraft/table.py:26-29 (a format
# table: it has to be identical to be the same format).
KVALUES_IQ4NL = np.array(
    [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113],
    dtype=np.float32,
)
IQ4_BLOCK_BYTES = 18


# ----------------------------------------------------------------------------
# bf16 / fp16 bit helpers
# ----------------------------------------------------------------------------

def f32_to_bf16_bits(x) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit pattern (uint16).  NaN stays NaN."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        rounded = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded)
    return rounded


def bf16_bits_to_f32(b) -> np.ndarray:
    """``engraft/replica/dequant.py:77-83``: bf16 -> f32 is ``bits << 16``."""
    b = np.ascontiguousarray(np.asarray(b, dtype=np.uint16))
    return (b.astype(np.uint32) << 16).view(np.float32)


# ----------------------------------------------------------------------------
# Q8_0 (split layout)
# ----------------------------------------------------------------------------

def dequant_q8_0(payload, scales) -> np.ndarray:
    """``[n, D]`` int8 + ``[n, D/32]`` fp16 -> ``[n, D]`` f32,
    ``y = f32(q) * f32(d)`` (``engraft/replica/dequant.py:86-93``)."""
    q = np.asarray(payload, dtype=np.int8)
    d = np.asarray(scales, dtype=np.float16).astype(np.float32)
    n, dim = q.shape
    qb = q.reshape(n, dim // BLOCK, BLOCK).astype(np.float32)
    with np.errstate(invalid="ignore"):  # inf scales times zero codes give NaN, as the format's arithmetic does
        return (qb * d[:, :, None]).reshape(n, dim)


def quant_q8_0(x) -> tuple[np.ndarray, np.ndarray]:
    """Build-defined requantisation rule (module docstring)."""
    x = np.asarray(x, dtype=np.float32)
    n, dim = x.shape
    xb = x.reshape(n, dim // BLOCK, BLOCK)
    amax = np.max(np.abs(xb), axis=2)
    d16 = (amax / np.float32(127.0)).astype(np.float32).astype(np.float16)
    d32 = d16.astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.rint(xb / d32[:, :, None])
    r = np.where(d32[:, :, None] == 0, 0, r)
    q = np.clip(r, -127, 127).astype(np.int8)
    return q.reshape(n, dim), d16


# ----------------------------------------------------------------------------
# MXFP8 (e4m3 + e8m0, split layout)
# ----------------------------------------------------------------------------

def e4m3_to_f32(bits) -> np.ndarray:
    """OCP e4m3 (``float8_e4m3fn``): bias 7, no inf, 0x7f/0xff = NaN,
    subnormals ``m * 2**-9``."""
    b = np.asarray(bits, dtype=np.uint8).astype(np.int32)
    s = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 0xF
    m = b & 0x7
    val = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    val = np.where((b & 0x7F) == 0x7F, np.nan, val)
    return (s * val).astype(np.float32)


def f32_to_e4m3(x) -> np.ndarray:
    """Round-to-nearest-even fp32 -> e4m3 bits; inputs must already lie in
    [-448, 448] (callers clamp).  Exhaustive over the representable grid: the
    code is the nearest grid value, ties to the even code."""
    x = np.asarray(x, dtype=np.float32)
    codes = np.arange(0, 0x7F, dtype=np.uint8)          # non-negative, non-NaN
    grid = e4m3_to_f32(codes).astype(np.float64)         # increasing
    a = np.abs(x).astype(np.float64)
    hi = np.clip(np.searchsorted(grid, a, side="left"), 0, len(grid) - 1)
    lo = np.clip(hi - 1, 0, len(grid) - 1)
    d_hi = np.abs(grid[hi] - a)
    d_lo = np.abs(a - grid[lo])
    pick_lo = (d_lo < d_hi) | ((d_lo == d_hi) & ((codes[lo] & 1) == 0))
    code = np.where(pick_lo, codes[lo], codes[hi]).astype(np.uint8)
    # the sign bit is kept even when the magnitude rounds to zero (-0 -> 0x80)
    return np.where(np.signbit(x), code | 0x80, code).astype(np.uint8)


def dequant_mxfp8(payload, scales) -> np.ndarray:
    """``[n, D]`` e4m3 bits + ``[n, D/32]`` e8m0 -> f32, ``y = v * 2**(e-127)``;
    e8m0 0xFF is NaN."""
    v = e4m3_to_f32(payload)
    e = np.asarray(scales, dtype=np.uint8).astype(np.int32)
    n, dim = v.shape
    with np.errstate(over="ignore", invalid="ignore"):  # large scales give inf, NaN scales NaN: the format's values
        scale = np.where(e == 255, np.nan, np.ldexp(np.float32(1.0), e - 127)).astype(np.float32)
        return (v.reshape(n, dim // BLOCK, BLOCK) * scale[:, :, None]).reshape(n, dim).astype(np.float32)


def quant_mxfp8(x) -> tuple[np.ndarray, np.ndarray]:
    """Build-defined MX quantisation (module docstring)."""
    x = np.asarray(x, dtype=np.float32)
    n, dim = x.shape
    xb = x.reshape(n, dim // BLOCK, BLOCK)
    amax = np.max(np.abs(xb), axis=2)
    ebits = ((amax.view(np.uint32) >> 23) & 0xFF).astype(np.int32)
    # floor(log2(amax)) - 8 for normal amax (subnormal amax -> -127 after the
    # clamp), plus one where amax * 2**-e would exceed 448: no block saturates
    e = np.where(amax > 0, ebits - 127, -127) - 8
    e = np.clip(e, -127, 127)
    over = (amax * np.ldexp(np.float32(1.0), -e).astype(np.float32)) > np.float32(448.0)
    e = np.clip(np.where(over, e + 1, e), -127, 127)
    scaled = xb * np.ldexp(np.float32(1.0), -e)[:, :, None].astype(np.float32)
    scaled = np.clip(scaled, -448.0, 448.0).astype(np.float32)
    q = f32_to_e4m3(scaled).reshape(n, dim)
    return q, (e + 127).astype(np.uint8)


# ----------------------------------------------------------------------------
# IQ4_NL (the reference's real table format)
# ----------------------------------------------------------------------------

def dequant_iq4nl(raw) -> np.ndarray:
    """``uint8 [n, 18*nb] -> f32 [n, 32*nb]``: ``engraft/table.py:147-169``.
    Block = fp16 d then 16 nibble bytes; ``y[j] = d*kv[qs[j] & 0xF]``,
    ``y[j+16] = d*kv[qs[j] >> 4]``."""
    raw = np.asarray(raw, dtype=np.uint8)
    n, nbytes = raw.shape
    nb = nbytes // IQ4_BLOCK_BYTES
    blocks = raw.reshape(n, nb, IQ4_BLOCK_BYTES)
    d = blocks[:, :, 0:2].copy().view(np.float16).astype(np.float32).reshape(n, nb)
    qs = blocks[:, :, 2:]
    y = np.concatenate([KVALUES_IQ4NL[qs & 0x0F], KVALUES_IQ4NL[qs >> 4]], axis=2)
    with np.errstate(invalid="ignore"):  # inf scales times zero codes give NaN, as the format's arithmetic does
        return (y * d[:, :, None]).reshape(n, nb * BLOCK).astype(np.float32)


def row_is_zero(raw) -> np.ndarray:
    """``engraft/table.py:172-183``: True iff every block's fp16 scale bit
    pattern is 0x0000 (a -0.0 scale counts as non-zero)."""
    raw = np.asarray(raw, dtype=np.uint8)
    n, nbytes = raw.shape
    blocks = raw.reshape(n, nbytes // IQ4_BLOCK_BYTES, IQ4_BLOCK_BYTES)
    return np.all((blocks[:, :, 0] == 0) & (blocks[:, :, 1] == 0), axis=1)


# ----------------------------------------------------------------------------
# GGML wire blocks (read_rows_raw's byte form)
# ----------------------------------------------------------------------------

WIRE_BLOCK_BYTES = {"f32": 4, "bf16": 2, "q8_0": 34, "iq4_nl": 18, "mxfp8": 33}


def wire_rows(fmt: str, payload, scales=None) -> np.ndarray:
    """Split-layout rows as GGML wire bytes ``uint8 [n, blocks*block_bytes]``:
    per 32-value block the scale (fp16 ``d`` for Q8_0, the e8m0 byte for
    MXFP8) then the 32 values; BF16/F32 rows are their own bytes; IQ4_NL rows
    are wire blocks already."""
    if fmt in ("bf16", "f32", "iq4_nl"):
        p = np.ascontiguousarray(payload)
        return p.view(np.uint8).reshape(p.shape[0], -1)
    q = np.ascontiguousarray(payload).view(np.uint8)
    n, dim = q.shape
    sc = np.ascontiguousarray(scales).view(np.uint8).reshape(n, dim // BLOCK, -1)
    return np.concatenate([sc, q.reshape(n, dim // BLOCK, BLOCK)], axis=2).reshape(n, -1)


def dequant_wire(fmt: str, blocks) -> np.ndarray:
    """``uint8 [..., block_bytes]`` wire blocks -> ``f32 [..., values]``
    (``engraft/replica/dequant.py:71-93, 127-147``): split back into payload
    and scales and decoded by the split-layout functions above."""
    b = np.ascontiguousarray(np.asarray(blocks, dtype=np.uint8))
    lead = b.shape[:-1]
    assert b.shape[-1] == WIRE_BLOCK_BYTES[fmt]
    b = b.reshape(-1, b.shape[-1])
    if fmt == "f32":
        out = b.copy().view(np.float32)
    elif fmt == "bf16":
        out = bf16_bits_to_f32(b.copy().view(np.uint16))
    elif fmt == "iq4_nl":
        out = dequant_iq4nl(b)
    elif fmt == "q8_0":
        out = dequant_q8_0(b[:, 2:].copy().view(np.int8), b[:, :2].copy().view(np.float16))
    else:
        out = dequant_mxfp8(b[:, 1:].copy(), b[:, :1].copy())
    return out.reshape(*lead, out.shape[-1])


# ----------------------------------------------------------------------------
# generic dispatch
# ----------------------------------------------------------------------------

def dequant(fmt: str, payload, scales=None) -> np.ndarray:
    if fmt == "bf16":
        return bf16_bits_to_f32(np.asarray(payload).view(np.uint16))
    if fmt == "q8_0":
        return dequant_q8_0(payload, scales)
    if fmt == "mxfp8":
        return dequant_mxfp8(payload, scales)
    if fmt == "iq4_nl":
        return dequant_iq4nl(payload)
    if fmt == "f32":
        return np.asarray(payload, dtype=np.float32)
    raise ValueError(f"unknown row format {fmt!r}")
