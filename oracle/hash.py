"""Oracle: the n-gram row hash (TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py).

Two independent restatements of the reference hash:

* ``ngram_addresses_scalar`` -- literal, per position, Python big ints, exactly
  the control flow of ``engraft/table.py:111-144`` (identical copy in
  ``engraft/testing/fake_table.py:41-66``).  Pure-Python loops: small cases only.
* ``ngram_rows_np`` -- vectorized numpy uint64, the formulation of
  ``engraft/damage.py:68-104`` generalised from ``ngram_size == 3`` to any
  ``ngram_size`` and extended with segment starts (the hash context of a
  position never reaches before its segment start, ``engraft/replica/seq.py:
  392-399`` with ``pack.pack_fragments`` segments, ``engraft/replica/pack.py:
  99-161``).

Pinning (tests/test_oracle_hash.py):
  * scalar == vectorized on the reference's own cross-check corpus
    (``tests/test_damage.py:19-61``: FakeTable(seed=7) multipliers, 20,000 tokens
    uniform over 50 ids, EOS every 200);
  * hand-computed identities of ``tests/test_table.py:66-94`` (no-EOS trigram,
    EOS substitution for a missing predecessor) and range check ``:97-102``;
  * EOS special cases the closed form fixes (EOS at t does not cut; EOS at t-1
    cuts t-2 even when t-2 is a regular token; start of sequence/segment);
  * unsigned-modulus edge values (mixed >= 2**63, multiples of p, p-1, 2**64-1)
    against Python's arbitrary-precision ``%``.
"""
from __future__ import annotations

import dataclasses

import numpy as np

MASK64 = (1 << 64) - 1


@dataclasses.dataclass(frozen=True)
class HashSpec:
    """Hash parameters of one table layer (``engraft/table.py:60-67``,
    ``engraft/replica/hparams.py:60-70``): one multiplier per context slot
    (``ctx[0]`` = current token), ``heads_per_ngram`` heads per order
    n = 2..ngram_size, head h of order n = ``(n-2)*heads_per_ngram + g``."""

    eos_token_id: int
    ngram_size: int
    heads_per_ngram: int
    layer_multipliers: tuple
    head_vocab_sizes: tuple
    head_offsets: tuple
    # Optional per-head multipliers ``[n_heads][ngram_size]`` (BASELINE's
    # synthetic tables seed the multipliers per slot and head).  ``None`` is the
    # reference's own mode: every head of an order shares ``layer_multipliers``.
    head_multipliers: tuple | None = None

    def mult(self, h: int) -> tuple:
        if self.head_multipliers is None:
            return tuple(self.layer_multipliers)
        return tuple(self.head_multipliers[h])

    @property
    def n_heads(self) -> int:
        return len(self.head_vocab_sizes)


def ngram_addresses_scalar(spec: HashSpec, tokens: list[int]) -> list[list[int]]:
    """Local row per head for every position of ``tokens``.

    Literal restatement of ``PleTable.ngram_addresses`` (``engraft/table.py:
    111-144``): ``ctx = [x_t, x_{t-1}, ...]``; a missing predecessor or an EOS met
    while walking back sets that slot and every older one to the EOS id
    (``:121-131``); the current token's own EOS never cuts.  For each order
    n = 2..ngram_size, ``mixed = XOR_{j<n} (ctx[j]*m[j] mod 2**64)`` (``:135-138``)
    and the order's heads take ``mixed % head_vocab_sizes[h]`` (``:139-142``)."""
    m = spec.layer_multipliers
    eos = spec.eos_token_id
    out: list[list[int]] = []
    for t in range(len(tokens)):
        ctx = [tokens[t]]
        cut = False
        for s in range(1, spec.ngram_size):
            pos = t - s
            tok = tokens[pos] if (pos >= 0 and not cut) else None
            if tok is None or tok == eos:
                cut = True
                tok = eos
            ctx.append(tok)
        rows_t: list[int] = []
        for n in range(2, spec.ngram_size + 1):
            base = (n - 2) * spec.heads_per_ngram
            if spec.head_multipliers is None:
                mixed = (ctx[0] * m[0]) & MASK64
                for j in range(1, n):
                    mixed ^= (ctx[j] * m[j]) & MASK64
                mixed &= MASK64
                for g in range(spec.heads_per_ngram):
                    rows_t.append(mixed % spec.head_vocab_sizes[base + g])
            else:  # generalised mode: the same formula with the head's own multipliers
                for g in range(spec.heads_per_ngram):
                    mh = spec.head_multipliers[base + g]
                    mixed = 0
                    for j in range(n):
                        mixed ^= (ctx[j] * mh[j]) & MASK64
                    rows_t.append(mixed % spec.head_vocab_sizes[base + g])
        out.append(rows_t)
    return out


def local_to_global(spec: HashSpec, h: int, row_local: int) -> int:
    """``engraft/lens.py:108-110``: global row = head offset + local row."""
    return int(spec.head_offsets[h]) + int(row_local)


def segment_starts(n: int, seq_len: int | None = None, seg_start=None) -> np.ndarray:
    """Start index (in the flat token array) of the segment of every position.

    ``seg_start`` given: used as is.  Otherwise independent rows of ``seq_len``
    positions (a ``[B, T]`` batch flattened; every row is its own sequence).
    ``seq_len=None``: one sequence."""
    if seg_start is not None:
        s = np.asarray(seg_start, dtype=np.int64)
        assert s.shape == (n,)
        return s
    idx = np.arange(n, dtype=np.int64)
    if seq_len is None:
        return np.zeros(n, dtype=np.int64)
    return (idx // seq_len) * seq_len


def seg_starts_from_segment_ids(segment_ids) -> np.ndarray:
    """Per-position segment start from contiguous increasing ``segment_ids``
    (``engraft/replica/seq.py:299-322``: the first index at which each id
    appears)."""
    seg = np.asarray(segment_ids)
    n = seg.shape[0]
    out = np.zeros(n, dtype=np.int64)
    first: dict[int, int] = {}
    for i, v in enumerate(seg.tolist()):
        if v not in first:
            first[v] = i
        out[i] = first[v]
    return out


def ngram_rows_np(spec: HashSpec, tokens, seq_len: int | None = None, seg_start=None,
                  global_ids: bool = True) -> np.ndarray:
    """``[n, n_heads]`` int64 rows for every position of the flat ``tokens``.

    Vectorized numpy-uint64 restatement of ``engraft/damage.py:68-104``
    (``x1 = eos`` where invalid, ``cut1 = ~valid1 | x1 == eos``,
    ``x2 = where(cut1, eos, x2_raw)``), generalised to ``ngram_size`` slots by
    carrying ``cut`` down the context, and with the validity test
    ``pos >= segment start`` instead of ``pos >= 0``.  numpy wraps uint64
    products modulo 2**64 like the scalar version's masking."""
    tok = np.asarray(tokens).astype(np.int64).reshape(-1)
    n = tok.shape[0]
    eos = np.uint64(spec.eos_token_id & MASK64)
    starts = segment_starts(n, seq_len, seg_start)
    idx = np.arange(n, dtype=np.int64)
    u = tok.astype(np.uint64)

    ctx = [u]
    cut = np.zeros(n, dtype=bool)
    for s in range(1, spec.ngram_size):
        pos = idx - s
        valid = pos >= starts
        raw = np.where(valid, u[np.clip(pos, 0, None)], eos)
        cut = cut | (~valid) | (raw == eos)
        ctx.append(np.where(cut, eos, raw))

    out = np.empty((n, spec.n_heads), dtype=np.int64)
    for order in range(2, spec.ngram_size + 1):
        base = (order - 2) * spec.heads_per_ngram
        for g in range(spec.heads_per_ngram):
            h = base + g
            mult = [np.uint64(int(m) & MASK64) for m in spec.mult(h)]
            mixed = ctx[0] * mult[0]
            for j in range(1, order):
                mixed = mixed ^ (ctx[j] * mult[j])
            local = (mixed % np.uint64(spec.head_vocab_sizes[h])).astype(np.int64)
            out[:, h] = local + (int(spec.head_offsets[h]) if global_ids else 0)
    return out
