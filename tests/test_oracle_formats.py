"""Pins the CPU oracle's row formats and the synthetic generator (no GPU)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import formats as F
from oracle import synth


def test_bf16_rounding_matches_torch():
    """fp32 -> bf16 RNE against torch's own conversion (library routine),
    including ties, carries into the exponent, inf, denormals."""
    rng = np.random.default_rng(0)
    x = rng.standard_normal(100_000).astype(np.float32) * np.float32(3.0)
    specials = np.array([0.0, -0.0, 1.0, np.inf, -np.inf, 1e-40, -1e-40, 3.0e38, 65504.0,
                         np.float32(1.00390625), np.float32(1.01171875)], dtype=np.float32)
    ties = (np.arange(1, 2000, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    x = np.concatenate([x, specials, ties])
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(F.f32_to_bf16_bits(x), ref)
    back = torch.from_numpy(ref.view(np.int16)).view(torch.bfloat16).float().numpy()
    assert np.array_equal(F.bf16_bits_to_f32(ref), back)
    nan = F.f32_to_bf16_bits(np.array([np.nan], dtype=np.float32))
    assert np.isnan(F.bf16_bits_to_f32(nan)).all()


def test_q8_0_dequant_closed_form():
    """engraft/replica/dequant.py:86-93: y = f32(int8) * f32(fp16 d)."""
    q = np.arange(-127, 129, dtype=np.int64)[:128].clip(-128, 127).astype(np.int8).reshape(1, 128)
    d = np.array([[0.5, -0.25, 2.0 ** -14, 3.0]], dtype=np.float16)
    y = F.dequant_q8_0(q, d)
    for b in range(4):
        np.testing.assert_array_equal(y[0, b * 32:(b + 1) * 32],
                                      q[0, b * 32:(b + 1) * 32].astype(np.float64) * float(d[0, b]))


def test_q8_0_requant_bounds_and_extremes():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((512, 128)) * 0.02).astype(np.float32)
    x[3, :32] = 0.0                      # all-zero block
    x[4, 32:64] = 1e-5                   # subnormal fp16 scale
    x[5, 64:96] = 1e-7                   # scale underflows fp16: the block quantises to 0
    q, d = F.quant_q8_0(x)
    assert d[5, 2] == 0 and np.all(q[5, 64:96] == 0)
    x[5, 64:96] = 0.0
    y = F.dequant_q8_0(q, d)
    d32 = np.repeat(d.astype(np.float32), 32, axis=1)
    # |y - x| <= d/2 except where the clamp at 127 bites (amax/d slightly > 127)
    err = np.abs(y - x)
    assert np.all((err <= d32 / 2 * (1 + 1e-6)) | (np.abs(q.astype(np.int32)) == 127))
    assert np.all(np.abs(q.astype(np.int32)) <= 127)
    assert np.all(q[3, :32] == 0) and np.all(d[3, 0] == 0)
    # the block maximum maps to +-127
    blocks = np.abs(x.reshape(512, 4, 32))
    amax_idx = blocks.argmax(axis=2)
    qb = np.abs(q.reshape(512, 4, 32).astype(np.int32))
    nz = d != 0
    assert np.all(np.take_along_axis(qb, amax_idx[:, :, None], 2)[:, :, 0][nz] == 127)


def test_q8_0_requant_exhaustive_small_blocks():
    """Every block whose values are k*s for integers |k| <= 127 with max |k| = 127
    and an fp16-exact s round-trips exactly."""
    rng = np.random.default_rng(2)
    k = rng.integers(-127, 128, size=(2000, 32))
    k[:, 0] = 127 * np.where(rng.random(2000) < 0.5, 1, -1)
    s = np.float16(2.0 ** -9) * rng.integers(1, 64, size=(2000, 1)).astype(np.float16)
    x = (k * s.astype(np.float32)).astype(np.float32)
    q, d = F.quant_q8_0(x)
    np.testing.assert_array_equal(F.dequant_q8_0(q, d), x)


def test_e4m3_decode_matches_torch_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = F.e4m3_to_f32(codes)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    assert np.array_equal(got[ok], ref[ok])
    assert np.array_equal(np.signbit(got[ok]), np.signbit(ref[ok]))


def test_e4m3_encode_matches_torch():
    """RNE fp32 -> e4m3 over [-448, 448] against torch's float8_e4m3fn cast."""
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.uniform(-448, 448, 50_000), rng.standard_normal(50_000) * 0.05,
                        rng.standard_normal(20_000) * 2.0 ** -8]).astype(np.float32)
    grid = F.e4m3_to_f32(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)
    mids = ((grid[1:] + grid[:-1]) / 2).astype(np.float32)  # exact ties
    x = np.concatenate([x, mids, -mids, np.array([0.0, -0.0, 448.0, -448.0], dtype=np.float32)])
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(F.f32_to_e4m3(x), ref)


def test_mxfp8_quant_roundtrip():
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((256, 128)) * 0.02).astype(np.float32)
    x[0, :32] = 0.0
    q, e = F.quant_mxfp8(x)
    y = F.dequant_mxfp8(q, e)
    assert np.all(y[0, :32] == 0)
    # e4m3 keeps 3 mantissa bits: relative error <= 2**-4 on normal values
    blocks = np.abs(x.reshape(256, 4, 32)).max(axis=2)
    big = (np.abs(x) >= np.repeat(blocks, 32, axis=1) * 2.0 ** -6) & (np.abs(x) > 0)
    rel = np.abs(y - x)[big] / np.abs(x)[big]
    assert rel.max() <= 2.0 ** -4 + 1e-7
    # the shared exponent is the smallest that keeps the block maximum <= 448
    amax = np.abs(x).reshape(256, 4, 32).max(axis=2)
    ex = e.astype(np.int32) - 127
    assert np.all((amax * 2.0 ** -ex)[1:] <= 448) and np.all((amax * 2.0 ** (1 - ex))[1:] > 448)


def test_iq4nl_dequant_closed_form_and_nibble_order():
    """engraft/table.py:147-169: y[j] = d*kv[qs[j] & 0xF], y[j+16] = d*kv[qs[j] >> 4]
    (swapping the nibble halves fails)."""
    raw = np.zeros((1, 90), dtype=np.uint8)
    for b in range(5):
        d = np.array([0.5 * (b + 1)], dtype=np.float16).view(np.uint8)
        raw[0, b * 18:b * 18 + 2] = d
        raw[0, b * 18 + 2:b * 18 + 18] = [(j & 15) | (((15 - j) & 15) << 4) for j in range(16)]
    y = F.dequant_iq4nl(raw)
    for b in range(5):
        d = 0.5 * (b + 1)
        for j in range(16):
            assert y[0, b * 32 + j] == np.float32(d * F.KVALUES_IQ4NL[j])
            assert y[0, b * 32 + 16 + j] == np.float32(d * F.KVALUES_IQ4NL[15 - j])


def test_row_is_zero_reference_vector():
    """tests/test_table.py:57-63, plus the -0.0-scale case (0x8000 is non-zero)."""
    raw = np.zeros((4, 90), dtype=np.uint8)
    raw[1, 0] = 1
    raw[2, 36] = 0
    raw[3, 19] = 0x80  # block 1 scale = -0.0
    assert F.row_is_zero(raw).tolist() == [True, False, True, False]


def test_splitmix64_published_sequence():
    """SplitMix64 seeded with 0 (Steele/Lea/Flood; Vigna's splitmix64.c):
    outputs 0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F."""
    g = synth.GOLDEN
    z = synth.mix64(np.array([0, g, (2 * g) % 2**64], dtype=np.uint64))
    assert [int(v) for v in z] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_quantile_table_is_normal():
    q = synth.quantile_table(1.0)
    assert q.shape == (16384,) and np.all(np.diff(q) > 0)
    assert abs(q.mean()) < 1e-6 and abs(q.std() - 1.0) < 2e-3
    vals = synth.synth_values(0, np.arange(2000), 128, 0.02)
    assert abs(vals.std() - 0.02) < 5e-4 and abs(vals.mean()) < 5e-4


def test_zipf_tokens_distribution():
    t = synth.zipf_tokens(0, 200_000, 151_936, 1.1)
    assert t.min() >= 0 and t.max() < 151_936
    _, counts = np.unique(t, return_counts=True)
    top = np.sort(counts)[::-1]
    w = np.arange(1, 151_937, dtype=np.float64) ** -1.1
    p1 = 1.0 / w.sum()
    assert abs(top[0] / 200_000 - p1) < 0.01


def test_wire_blocks_known_answers():
    """Hand-computed wire blocks: Q8_0 with d = 0.5 (fp16 0x3800), BF16 1.0
    and -2.0, F32 bytes, IQ4_NL with d = 1 and nibble 0 / 15 (-127 / 113)."""
    q8 = np.zeros(34, np.uint8)
    q8[0:2] = [0x00, 0x38]
    q = np.zeros(32, np.int8)
    q[0], q[1], q[31] = -127, 1, 127
    q8[2:] = q.view(np.uint8)
    y = F.dequant_wire("q8_0", q8[None])[0]
    want = np.zeros(32, np.float32)
    want[0], want[1], want[31] = -63.5, 0.5, 63.5
    assert np.array_equal(y, want)
    bf = np.array([[0x80, 0x3F], [0x00, 0xC0]], np.uint8)
    assert F.dequant_wire("bf16", bf).tolist() == [[1.0], [-2.0]]
    assert F.dequant_wire("f32", np.array([[0, 0, 0x80, 0xBF]], np.uint8)).tolist() == [[-1.0]]
    iq = np.zeros(18, np.uint8)
    iq[0:2] = [0x00, 0x3C]  # fp16 1.0
    iq[2] = 0xF0            # value 0: low nibble 0, value 16: high nibble 15
    y = F.dequant_wire("iq4_nl", iq[None])[0]
    assert y[0] == -127.0 and y[16] == 113.0 and y[1] == -127.0


@pytest.mark.parametrize("fmt", ["q8_0", "mxfp8", "bf16", "f32", "iq4_nl"])
def test_wire_blocks_agree_with_split_layout(fmt):
    """The wire form of split-layout rows decodes to the split layout's own
    values (the two layouts hold the same rows)."""
    rng = np.random.default_rng(5)
    n, dim = 7, 96
    if fmt == "q8_0":
        payload = rng.integers(-127, 128, (n, dim)).astype(np.int8)
        scales = (rng.standard_normal((n, dim // 32)) * 0.01).astype(np.float16)
    elif fmt == "mxfp8":
        payload = rng.integers(0, 256, (n, dim)).astype(np.uint8)
        scales = rng.integers(100, 150, (n, dim // 32)).astype(np.uint8)
    elif fmt == "bf16":
        payload, scales = rng.integers(0, 1 << 16, (n, dim)).astype(np.uint16), None
    elif fmt == "f32":
        payload, scales = rng.standard_normal((n, dim)).astype(np.float32), None
    else:
        payload, scales = rng.integers(0, 256, (n, dim // 32 * 18)).astype(np.uint8), None
        payload.reshape(n, -1, 18)[:, :, 1] &= 0x3F  # finite scales
    wire = F.wire_rows(fmt, payload, scales)
    got = F.dequant_wire(fmt, wire.reshape(n, -1, F.WIRE_BLOCK_BYTES[fmt])).reshape(n, dim)
    want = F.dequant(fmt, payload, scales)
    assert np.array_equal(got, want, equal_nan=True)
