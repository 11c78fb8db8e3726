"""Seeded synthetic inputs of the benchmark's configurations.

* ``hash_params``  -- the benchmark's synthetic table addressing: the table is
  split evenly between the ``(ngram_size-1)*heads_per_ngram`` heads, and every
  head has its own seeded odd 64-bit multiplier per context slot (the
  benchmark's "16 fixed seeded 64-bit odd multipliers, mod rows").  EOS, which
  the benchmark's definition leaves open, is 151,643 (Qwen ``<|endoftext|>``).
* ``table``        -- a seeded table generated in place on the device
  (``eg_synth_table``): value j of row r is a normal quantile picked by
  SplitMix64 of ``(seed, r, j)``, quantised with the format's rule.
* ``zipf_tokens`` / ``uniform_tokens`` -- token streams (rank k drawn with
  probability proportional to ``k**-s`` by the inverse CDF, ranks mapped to
  ids by a seeded permutation).
"""
from __future__ import annotations

import numpy as np
import torch

from .table import DeviceTable

QWEN_EOS = 151_643


def odd_multipliers(seed: int, count: int) -> list[int]:
    rng = np.random.default_rng(seed)
    return [int(v) | 1 for v in rng.integers(1, 2 ** 63, size=count, dtype=np.int64, endpoint=False)]


def hash_params(n_rows: int, seed: int, ngram_size: int = 3, heads_per_ngram: int = 8, eos: int = QWEN_EOS,
                row0: int = 0) -> dict:
    n_heads = (ngram_size - 1) * heads_per_ngram
    per = n_rows // n_heads
    mults = odd_multipliers(seed, n_heads * ngram_size)
    head_mult = [mults[h * ngram_size:(h + 1) * ngram_size] for h in range(n_heads)]
    return dict(eos_token_id=eos, ngram_size=ngram_size, heads_per_ngram=heads_per_ngram,
                layer_multipliers=head_mult[0], head_vocab_sizes=[per] * n_heads,
                head_offsets=[row0 + h * per for h in range(n_heads)], head_multipliers=head_mult)


def table(fmt: str, n_rows: int, dim: int, *, seed: int, hash_seed: int, sigma: float = 0.02,
          ngram_size: int = 3, heads_per_ngram: int = 8, device="cuda") -> DeviceTable:
    hp = hash_params(n_rows, hash_seed, ngram_size=ngram_size, heads_per_ngram=heads_per_ngram)
    return DeviceTable.synthetic(fmt, n_rows, dim, seed=seed, sigma=sigma, device=device, **hp)


def zipf_tokens(seed: int, n: int, vocab: int, s: float = 1.1) -> np.ndarray:
    rng = np.random.default_rng(seed)
    perm = rng.permutation(vocab).astype(np.int64)
    w = np.arange(1, vocab + 1, dtype=np.float64) ** (-s)
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    rank = np.minimum(np.searchsorted(cdf, rng.random(n), side="right"), vocab - 1)
    return perm[rank]


def uniform_tokens(seed: int, n: int, vocab: int) -> np.ndarray:
    return np.random.default_rng(seed).integers(0, vocab, size=n, dtype=np.int64)


def residual(n: int, width: int, seed: int, device="cuda", std: float = 1.0) -> torch.Tensor:
    """bf16 ``[n, width]`` ~ N(0, std**2) from torch's seeded device generator."""
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn((n, width), generator=g, device=device, dtype=torch.float32)
    if std != 1.0:
        x.mul_(std)
    return x.to(torch.bfloat16)
