"""Oracle: gather + dequant + overlay substitution + residual add
(TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py).

* ``gather``        -- ``RowSet.from_position`` per position, vectorized
  (``engraft/lens.py:126-136``): the ``n_heads`` rows of every position,
  dequantised, concatenated head after head (``engraft/replica/seq.py:444``
  reshape ``[n, n_heads*row_len]``).
* ``substitute``    -- overlay rows replace the base rows whose global id is in
  the overlay, every other row stays bit-identical
  (``engraft/replica/model.py:473-495``; ``engraft/replica/seq.py:412-441``
  int-key branch).
* ``residual_add``  -- BASELINE's consumer: ``bf16_rne(f32(residual) + emb_0
  [+ emb_1 ...])``, the layers added in order, fp32 accumulate.

Pinning (tests/test_oracle_forward_backward.py): the substitution invariants of
``tests/test_replica_graft.py:43-70`` (present rows replaced, absent rows
bit-identical, empty overlay == plain gather), the fp32-add-then-RNE rule
against torch's ``.to(torch.bfloat16)`` (library routine), and the gather
against the per-position scalar ``RowSet`` loop on small cases.
"""
from __future__ import annotations

import numpy as np

from oracle import formats as F
from oracle import hash as H


def gather(rows, fetch) -> np.ndarray:
    """``rows`` int ``[P, Hh]`` global ids, ``fetch(ids) -> f32 [m, D]``;
    returns f32 ``[P, Hh*D]`` (head-major concatenation)."""
    rows = np.asarray(rows, dtype=np.int64)
    p, hh = rows.shape
    vals = fetch(rows.reshape(-1))
    d = vals.shape[1]
    return vals.reshape(p, hh * d)


def substitute(emb, rows, ov_ids, ov_rows) -> tuple[np.ndarray, int]:
    """Replace, in ``emb [P, Hh*D]``, every head slot whose global row is in
    the sorted overlay ``ov_ids`` by the matching ``ov_rows`` f32 vector.
    Returns the new emb and the hit count (``n_id_hits``)."""
    emb = np.array(emb, dtype=np.float32, copy=True)
    rows = np.asarray(rows, dtype=np.int64)
    ov_ids = np.asarray(ov_ids, dtype=np.int64)
    p, hh = rows.shape
    d = emb.shape[1] // hh
    if ov_ids.size == 0:
        return emb, 0
    flat = rows.reshape(-1)
    pos = np.searchsorted(ov_ids, flat)
    posc = np.clip(pos, 0, ov_ids.size - 1)
    hit = ov_ids[posc] == flat
    e3 = emb.reshape(p * hh, d)
    e3[hit] = np.asarray(ov_rows, dtype=np.float32)[posc[hit]]
    return e3.reshape(p, hh * d), int(hit.sum())


def residual_add(residual_bits, embs) -> np.ndarray:
    """bf16 bits out of ``f32(residual) + emb_0 + emb_1 + ...`` (fp32, in order)."""
    acc = F.bf16_bits_to_f32(residual_bits).astype(np.float32)
    for e in embs:
        acc = (acc + np.asarray(e, dtype=np.float32)).astype(np.float32)
    return F.f32_to_bf16_bits(acc)


def forward(spec: H.HashSpec, tokens, fetch, residual_bits=None, seq_len=None, seg_start=None,
            overlay=None):
    """One table layer end to end: hash -> gather -> substitute [-> add].

    Returns ``(rows [P, Hh] int64, emb f32 [P, W], out bf16 bits or None)``."""
    rows = H.ngram_rows_np(spec, tokens, seq_len=seq_len, seg_start=seg_start)
    emb = gather(rows, fetch)
    if overlay is not None:
        emb, _ = substitute(emb, rows, overlay[0], overlay[1])
    out = residual_add(residual_bits, [emb]) if residual_bits is not None else None
    return rows, emb, out


def table_fetch(fmt: str, payload, scales=None):
    """``fetch`` over an explicit in-memory table (rows indexed by global id)."""
    payload = np.asarray(payload)
    scales = None if scales is None else np.asarray(scales)

    def fetch(ids):
        ids = np.asarray(ids, dtype=np.int64)
        return F.dequant(fmt, payload[ids], None if scales is None else scales[ids])

    return fetch
