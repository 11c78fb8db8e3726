"""Oracle: seeded synthetic inputs (TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py).

The device generator (``eg_synth_table`` in the HIP library) must produce the
same bytes as ``synth_rows`` for every row, so that the CPU side can regenerate
any row of a 43.5 GB device table from its id alone.

Value ``j`` of global row ``r`` (``D`` values per row):

    z   = mix64(seed * 0xD1B54A32D192ED03 + r * D + j)      (all mod 2**64)
    x   = Q[z >> 50]

``mix64`` is the SplitMix64 output function (Steele, Lea, Flood, "Fast
splittable pseudorandom number generators", OOPSLA 2014), and ``Q`` the
16,384-entry table of normal quantiles ``Q[i] = f32(sigma * Phi^-1((i+0.5)/16384))``
computed in float64 (``statistics.NormalDist``).  Rows are then quantised with
the format's rule from ``oracle.formats`` (bf16: RNE).

Tokens: ``zipf_tokens`` draws ranks with probability ``k**-s / H`` (k = 1..V)
through the inverse CDF and maps them to ids with a seeded permutation
(BASELINE configs 1-4); ``uniform_tokens`` draws ids uniformly (config 0).
"""
from __future__ import annotations

import statistics

import numpy as np

from oracle import formats as F

GOLDEN = 0x9E3779B97F4A7C15
SEED_MUL = 0xD1B54A32D192ED03
_M1 = 0xBF58476D1CE4E5B9
_M2 = 0x94D049BB133111EB
QTABLE_SIZE = 16384


def mix64(z) -> np.ndarray:
    """SplitMix64 output function on uint64 arrays (wrapping arithmetic)."""
    z = np.asarray(z, dtype=np.uint64) + np.uint64(GOLDEN)
    z = (z ^ (z >> np.uint64(30))) * np.uint64(_M1)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(_M2)
    return z ^ (z >> np.uint64(31))


def quantile_table(sigma: float) -> np.ndarray:
    nd = statistics.NormalDist(0.0, 1.0)
    q = np.array([nd.inv_cdf((i + 0.5) / QTABLE_SIZE) for i in range(QTABLE_SIZE)], dtype=np.float64)
    return (q * sigma).astype(np.float32)


_QCACHE: dict[float, np.ndarray] = {}


def _qtable(sigma: float) -> np.ndarray:
    if sigma not in _QCACHE:
        _QCACHE[sigma] = quantile_table(sigma)
    return _QCACHE[sigma]


def synth_values(seed: int, rows, dim: int, sigma: float) -> np.ndarray:
    """f32 ``[len(rows), dim]`` pre-quantisation values of the given global rows."""
    rows = np.asarray(rows, dtype=np.uint64).reshape(-1)
    base = np.uint64((seed * SEED_MUL) & ((1 << 64) - 1))
    idx = base + rows[:, None] * np.uint64(dim) + np.arange(dim, dtype=np.uint64)[None, :]
    z = mix64(idx)
    return _qtable(sigma)[(z >> np.uint64(50)).astype(np.int64)]


def synth_rows(fmt: str, seed: int, rows, dim: int, sigma: float):
    """The stored bytes of the given rows: ``(payload, scales)`` (scales None for bf16/f32)."""
    x = synth_values(seed, rows, dim, sigma)
    if fmt == "bf16":
        return F.f32_to_bf16_bits(x), None
    if fmt == "q8_0":
        return F.quant_q8_0(x)
    if fmt == "mxfp8":
        return F.quant_mxfp8(x)
    if fmt == "f32":
        return x, None
    raise ValueError(f"synth_rows: unsupported format {fmt!r}")


def synth_dequant(fmt: str, seed: int, rows, dim: int, sigma: float) -> np.ndarray:
    payload, scales = synth_rows(fmt, seed, rows, dim, sigma)
    return F.dequant(fmt, payload, scales)


def zipf_tokens(seed: int, n: int, vocab: int, s: float = 1.1) -> np.ndarray:
    rng = np.random.default_rng(seed)
    perm = rng.permutation(vocab).astype(np.int64)
    w = np.arange(1, vocab + 1, dtype=np.float64) ** (-s)
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    u = rng.random(n)
    rank = np.minimum(np.searchsorted(cdf, u, side="right"), vocab - 1)
    return perm[rank]


def uniform_tokens(seed: int, n: int, vocab: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return rng.integers(0, vocab, size=n, dtype=np.int64)


def odd_multipliers(seed: int, count: int) -> list[int]:
    """Seeded odd 64-bit multipliers (``engraft/testing/fake_table.py:33-36``
    draws ``integers(1, 2**61) | 1``; BASELINE's synthetic configs ask for full
    64-bit odd multipliers)."""
    rng = np.random.default_rng(seed)
    return [int(v) | 1 for v in rng.integers(1, 2 ** 63, size=count, dtype=np.int64, endpoint=False)]
