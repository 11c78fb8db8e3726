"""Pins the CPU oracle's n-gram hash (oracle/hash.py) against the reference's
own known-answer tests and the closed form (no GPU)."""
from __future__ import annotations

import numpy as np
import pytest

from oracle.hash import HashSpec, MASK64, ngram_addresses_scalar, ngram_rows_np, seg_starts_from_segment_ids
from tests.params import FAKE_EOS, fake_table_spec, reference_corpus, synthetic_spec, tiny_hparams_spec


def _mixed(ctx, mults, n):
    m = 0
    for j in range(n):
        m ^= (ctx[j] * mults[j]) & MASK64
    return m


def test_scalar_equals_vectorized_on_reference_corpus():
    """tests/test_damage.py:38-61: the scalar and the vectorized hash agree on
    FakeTable(seed=7) over 20,000 tokens (ids < 50, EOS every 200)."""
    spec = fake_table_spec(seed=7)
    tokens = reference_corpus()
    scalar = np.array(ngram_addresses_scalar(spec, tokens.tolist()), dtype=np.int64)
    vec_local = ngram_rows_np(spec, tokens, global_ids=False)
    assert np.array_equal(scalar, vec_local)
    vec_global = ngram_rows_np(spec, tokens)
    assert np.array_equal(vec_global, scalar + np.array(spec.head_offsets)[None, :])


@pytest.mark.parametrize("spec_fn", [tiny_hparams_spec, lambda: fake_table_spec(7)])
def test_hash_matches_hand_computed(spec_fn):
    """tests/test_table.py:66-81: mixed2 = (t0*m0)^(t1*m1), mixed3 = mixed2^(t2*m2)."""
    spec = spec_fn()
    m0, m1, m2 = spec.layer_multipliers[:3]
    t2, t1, t0 = 100, 200, 300
    mixed2 = ((t0 * m0) ^ (t1 * m1)) & MASK64
    mixed3 = (mixed2 ^ (t2 * m2)) & MASK64
    expected = [mixed2 % p for p in spec.head_vocab_sizes[0:8]] + [mixed3 % p for p in spec.head_vocab_sizes[8:16]]
    assert ngram_addresses_scalar(spec, [t2, t1, t0])[-1] == expected
    assert ngram_rows_np(spec, [t2, t1, t0], global_ids=False)[-1].tolist() == expected


def test_eos_replaces_missing_predecessor():
    """tests/test_table.py:84-94."""
    spec = tiny_hparams_spec()
    m0, m1 = spec.layer_multipliers[:2]
    mixed2 = ((42 * m0) ^ (FAKE_EOS * m1)) & MASK64
    exp2 = [mixed2 % p for p in spec.head_vocab_sizes[0:8]]
    assert ngram_addresses_scalar(spec, [42])[-1][0:8] == exp2
    assert ngram_rows_np(spec, [42], global_ids=False)[-1][0:8].tolist() == exp2


def test_addresses_in_range():
    """tests/test_table.py:97-102 (an EOS mid-sequence)."""
    spec = fake_table_spec(3)
    tokens = [10, 20000, 5, spec.eos_token_id, 99, 100000]
    for row in ngram_addresses_scalar(spec, tokens):
        assert len(row) == spec.n_heads
        for h, r in enumerate(row):
            assert 0 <= r < spec.head_vocab_sizes[h]


@pytest.mark.parametrize("tokens,t,ctx_expected", [
    ([7, 8, 9], 2, [9, 8, 7]),                      # plain trigram
    ([7, FAKE_EOS, 9], 2, [9, FAKE_EOS, FAKE_EOS]),  # EOS at t-1 cuts t-2 (7 is replaced)
    ([FAKE_EOS, 8, 9], 2, [9, 8, FAKE_EOS]),         # EOS at t-2 is kept as the EOS id
    ([7, 8, FAKE_EOS], 2, [FAKE_EOS, 8, 7]),         # the current token's EOS never cuts
    ([7, 8], 1, [8, 7, FAKE_EOS]),                   # missing t-2
    ([7], 0, [7, FAKE_EOS, FAKE_EOS]),               # missing t-1 and t-2
])
def test_eos_rule_closed_form(tokens, t, ctx_expected):
    """docs/mechanism.md:24-45: the context each position hashes.  Substituting
    0 instead of EOS, not carrying the cut, or cutting on the current token's
    EOS each fails one of these cases."""
    spec = fake_table_spec(11)
    m = spec.layer_multipliers
    mixed2 = _mixed(ctx_expected, m, 2)
    mixed3 = _mixed(ctx_expected, m, 3)
    exp = [mixed2 % p for p in spec.head_vocab_sizes[:8]] + [mixed3 % p for p in spec.head_vocab_sizes[8:]]
    assert ngram_addresses_scalar(spec, tokens)[t] == exp
    assert ngram_rows_np(spec, tokens, global_ids=False)[t].tolist() == exp


def test_unsigned_modulus_edge_values():
    """mixed = token (m = [1, 0]) walks the uint64 edge values: >= 2**63,
    2**64-1, multiples of p and p-1; a signed modulus or a truncation to 32
    bits fails here."""
    p = 4999
    spec = HashSpec(eos_token_id=FAKE_EOS, ngram_size=2, heads_per_ngram=3, layer_multipliers=(1, 0),
                    head_vocab_sizes=(p, 65521, 2**32 - 5), head_offsets=(0, p, p + 65521))
    vals = [0, 1, p - 1, p, 7 * p, 7 * p - 1, 2**32 - 1, 2**32, 2**63 - 1, 2**63, 2**63 + 1, 2**64 - 1,
            (2**64 - 1) - ((2**64 - 1) % p), 0xDEADBEEFCAFEBABE]
    tokens = [v - 2**64 if v >= 2**63 else v for v in vals]  # int64 bit patterns
    got = ngram_rows_np(spec, np.array(tokens, dtype=np.int64), global_ids=False)
    for i, v in enumerate(vals):
        assert got[i].tolist() == [v % q for q in spec.head_vocab_sizes]
    scalar = ngram_addresses_scalar(spec, [v for v in vals])
    assert np.array_equal(np.array(scalar, dtype=np.int64), got)


def test_per_head_multipliers_scalar_equals_vectorized():
    spec = synthetic_spec(n_rows=16 * 262_144, seed=5)
    rng = np.random.default_rng(2)
    tokens = rng.integers(0, 151_936, size=3000)
    tokens[::97] = spec.eos_token_id
    scalar = np.array(ngram_addresses_scalar(spec, tokens.tolist()), dtype=np.int64)
    assert np.array_equal(scalar, ngram_rows_np(spec, tokens, global_ids=False))
    # heads of one order do differ in this mode
    assert len(set(scalar[50, :8].tolist())) > 1


def test_four_gram_generalisation():
    """ngram_size = 4: the scalar literal form and the
    vectorized form agree, 24 heads."""
    spec = synthetic_spec(n_rows=24 * 1000, seed=9, ngram_size=4)
    rng = np.random.default_rng(3)
    tokens = rng.integers(0, 200, size=2000)
    tokens[::37] = spec.eos_token_id
    scalar = np.array(ngram_addresses_scalar(spec, tokens.tolist()), dtype=np.int64)
    assert scalar.shape == (2000, 24)
    assert np.array_equal(scalar, ngram_rows_np(spec, tokens, global_ids=False))


def test_segments_equal_isolated_fragments():
    """engraft/replica/seq.py:392-399: with segment_ids, position t hashes
    tokens[s(t):] -- the same as hashing each fragment on its own
    (tests/test_seq.py:54-57 segment layout)."""
    spec = fake_table_spec(1)
    tokens = [FAKE_EOS, 3, 5, 7, 2, FAKE_EOS, 9, 4, 6]
    seg_ids = [0, 0, 0, 0, 0, 1, 1, 1, 1]
    seg_start = seg_starts_from_segment_ids(seg_ids)
    got = ngram_rows_np(spec, tokens, seg_start=seg_start, global_ids=False)
    exp = ngram_addresses_scalar(spec, tokens[:5]) + ngram_addresses_scalar(spec, tokens[5:])
    assert got.tolist() == exp
    # batch rows of seq_len are independent sequences
    rng = np.random.default_rng(4)
    toks = rng.integers(0, 30, size=4 * 64)
    got = ngram_rows_np(spec, toks, seq_len=64, global_ids=False)
    exp = sum((ngram_addresses_scalar(spec, toks[i * 64:(i + 1) * 64].tolist()) for i in range(4)), [])
    assert got.tolist() == exp
