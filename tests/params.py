"""Hash/table parameter sets shared by the tests, the golden-vector script and
the benchmark (test and bench infrastructure)."""
from __future__ import annotations

import numpy as np

from oracle.hash import HashSpec
from oracle import synth

FAKE_EOS = 999_999_999  # engraft/testing/fake_table.py:20


def fake_table_spec(seed: int = 0, head_vocab_size: int = 5_000) -> HashSpec:
    """The parameters ``FakeTable(seed)`` draws (``engraft/testing/fake_table.py:
    23-37``): 16 heads of ``head_vocab_size`` rows, ngram 3, 8 heads per order,
    multipliers ``default_rng(seed).integers(1, 2**61) | 1`` per context slot
    (four of them).  Produced here by numpy's own generator, not by the
    reference's code."""
    rng = np.random.default_rng(seed)
    mults = tuple(int(rng.integers(1, 2**61)) | 1 for _ in range(4))
    return HashSpec(eos_token_id=FAKE_EOS, ngram_size=3, heads_per_ngram=8, layer_multipliers=mults,
                    head_vocab_sizes=tuple([head_vocab_size] * 16),
                    head_offsets=tuple(i * head_vocab_size for i in range(16)))


def tiny_hparams_spec() -> HashSpec:
    """``engraft/testing/fake_full_weights.py:51-53``: multipliers (1, 3, 5, 7),
    16 heads of 5,000 rows, EOS 999,999,999."""
    return HashSpec(eos_token_id=FAKE_EOS, ngram_size=3, heads_per_ngram=8, layer_multipliers=(1, 3, 5, 7),
                    head_vocab_sizes=tuple([5000] * 16), head_offsets=tuple(i * 5000 for i in range(16)))


def reference_corpus(n: int = 20_000, seed: int = 1, eos: int = FAKE_EOS, vocab: int = 50,
                     every: int = 200) -> np.ndarray:
    """``tests/test_damage.py:19-23``: uniform ids over ``vocab`` with an EOS every ``every``."""
    rng = np.random.default_rng(seed)
    tokens = rng.integers(0, vocab, size=n, dtype=np.int32)
    tokens[every - 1::every] = eos
    return tokens


def synthetic_spec(n_rows: int, seed: int, ngram_size: int = 3, heads_per_ngram: int = 8,
                   eos: int = 151_643, row0: int = 0) -> HashSpec:
    """BASELINE's synthetic tables: the table is split evenly between the
    ``(ngram_size-1)*heads_per_ngram`` heads and every head has its own seeded
    odd 64-bit multiplier per context slot.  EOS (not given by BASELINE) is
    151,643, the Qwen ``<|endoftext|>`` id."""
    n_heads = (ngram_size - 1) * heads_per_ngram
    per = n_rows // n_heads
    mults = synth.odd_multipliers(seed, n_heads * ngram_size)
    head_mult = tuple(tuple(mults[h * ngram_size:(h + 1) * ngram_size]) for h in range(n_heads))
    return HashSpec(eos_token_id=eos, ngram_size=ngram_size, heads_per_ngram=heads_per_ngram,
                    layer_multipliers=head_mult[0], head_vocab_sizes=tuple([per] * n_heads),
                    head_offsets=tuple(row0 + h * per for h in range(n_heads)), head_multipliers=head_mult)


# BASELINE.json configs (sizes only; the seeded data comes from oracle.synth)
CFG0 = dict(n_rows=4_194_304, dim=128, fmt="bf16", batch=1, seq=2048, vocab=151_936, width=2048, sigma=0.02)
CFG1 = dict(n_rows=320_000_000, dim=128, fmt="q8_0", batch=8, seq=2048, vocab=151_936, width=2048, sigma=0.02)
CFG4 = dict(n_rows=160_000_000, dim=128, fmt="mxfp8", batch=1, seq=32_768, vocab=129_280, width=3072, sigma=0.02,
            layers=2, ngram_size=4)
CFG3 = dict(n_rows=320_000_000, dim=128, fmt="q8_0", n_seq=256, ctx=3, overlay_rows=500_000, vocab=151_936,
            width=2048, sigma=0.02)
