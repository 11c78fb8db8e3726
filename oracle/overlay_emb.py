"""Oracle: the differentiable sequence overlay ``OverlayEmb`` and the
per-position ``ple_true_emb`` (TEST INFRASTRUCTURE ONLY -- see
oracle/__init__.py).

Literal per-position restatement of ``OverlayEmb.build``
(``engraft/replica/seq.py:372-444``), ``_gather_fragment_base``
(``:185-219``), ``overlay_key_len`` (``:222-234``) and
``Replica.ple_true_emb`` (``engraft/replica/model.py:473-495``): for every
position ``t`` the ``RowSet`` of ``tokens[s(t):]`` at ``t - s(t)``
(``s(t)`` = start of ``t``'s segment, 0 without ``segment_ids``), then, per
head, the long key ``(window, h)`` first (only when ``t_local >= K-1``), else
the global row, looked up in ``row_map``.  Pure-Python loops: small inputs
only.

Pinning (tests/test_oracle_overlay_emb.py): the invariants of
``tests/test_replica_graft.py:43-70`` (rows present in the map replaced, all
others bit-identical to the plain gather), the first-wins long key, the
segment rule against isolated per-fragment hashing
(``tests/test_seq.py:54-57``'s packing), ``n_key_hits + n_id_hits`` against a
brute-force count, and the gradient against torch's own autograd of
``index_put`` on the CPU (the library routine the reference differentiates).
"""
from __future__ import annotations

import numpy as np

from oracle import hash as H


def overlay_key_len(row_map: dict):
    """``engraft/replica/seq.py:222-234``: the common window length of the
    tuple keys, ``None`` without tuple keys; mixed lengths fail."""
    lengths = {len(key[0]) for key in row_map if isinstance(key, tuple)}
    if not lengths:
        return None
    assert len(lengths) == 1, f"overlay_key_len: long keys of different lengths in row_map: {lengths}"
    return next(iter(lengths))


def row_set(spec: H.HashSpec, tokens: list[int], t: int, fetch):
    """``RowSet.from_position`` (``engraft/lens.py:126-136``): global rows of
    position ``t`` (re-hashing the whole prefix, as the reference does) and
    their dequantised rows."""
    local = H.ngram_addresses_scalar(spec, list(tokens[:t + 1]))[t]
    rows = np.array([H.local_to_global(spec, h, r) for h, r in enumerate(local)], dtype=np.int64)
    return rows, fetch(rows)


def exclusive_rows_at_position(spec: H.HashSpec, tokens: list[int], n_positions: int, p: int, heads=None) -> set:
    """``engraft/replica/seq.py:924-941``: the rows of position ``p`` (among
    ``heads``) minus every row read at another position ``0..n_positions-1``,
    with the per-position ``row_set`` loop of the reference."""
    heads = heads if heads is not None else range(spec.n_heads)
    fetch0 = lambda r: None  # noqa: E731  (rows only)
    rows_p, _ = row_set(spec, tokens, p if p >= 0 else len(tokens) + p, fetch0)
    candidates = {int(rows_p[h]) for h in heads}
    for t in range(n_positions):
        if t == p:
            continue
        rows_t, _ = row_set(spec, tokens, t, fetch0)
        candidates -= {int(g) for g in rows_t}
    return candidates


def build_plan(spec: H.HashSpec, tokens: list[int], row_map: dict, n_positions: int, start: int = 0,
               segment_ids=None, fetch=None):
    """``OverlayEmb.build``'s cached part (``engraft/replica/seq.py:385-426``):
    ``(rows int64 [n, H], base f32 [n, H, D] or None, idx_t, idx_h, idx_r,
    n_key_hits, n_id_hits)`` for positions ``start..n_positions-1``."""
    key_len = overlay_key_len(row_map)
    seg_starts = None if segment_ids is None else H.seg_starts_from_segment_ids(segment_ids)
    n_heads = spec.n_heads
    rows_out = np.zeros((n_positions - start, n_heads), dtype=np.int64)
    base = [] if fetch is not None else None
    idx_t, idx_h, idx_r = [], [], []
    n_key_hits = n_id_hits = 0
    for t in range(start, n_positions):
        if seg_starts is not None:
            s_t = int(seg_starts[t])
            t_local = t - s_t
            seg_tokens = tokens[s_t:]
        else:
            t_local = t
            seg_tokens = tokens
        local = H.ngram_addresses_scalar(spec, list(seg_tokens[:t_local + 1]))[t_local]
        rows = [H.local_to_global(spec, h, r) for h, r in enumerate(local)]
        rows_out[t - start] = rows
        if base is not None:
            base.append(fetch(np.array(rows, dtype=np.int64)))
        window = None
        if key_len is not None and t_local >= key_len - 1:
            window = tuple(tokens[t - key_len + 1:t + 1])
        for h in range(n_heads):
            key = (window, h) if window is not None else None
            if key is not None and key in row_map:
                idx_t.append(t - start)
                idx_h.append(h)
                idx_r.append(row_map[key])
                n_key_hits += 1
                continue
            g = int(rows[h])
            if g in row_map:
                idx_t.append(t - start)
                idx_h.append(h)
                idx_r.append(row_map[g])
                n_id_hits += 1
    base_arr = None if base is None else (np.stack(base).astype(np.float32) if base else None)
    return rows_out, base_arr, idx_t, idx_h, idx_r, n_key_hits, n_id_hits


def build(spec, tokens, row_map, rows_var, n_positions, fetch, start=0, segment_ids=None):
    """The embedding ``[n, H*D]`` (``engraft/replica/seq.py:428-444``):
    ``base.index_put((idx_t, idx_h), rows_var[idx_r])``."""
    rows, base, idx_t, idx_h, idx_r, nk, ni = build_plan(spec, tokens, row_map, n_positions, start,
                                                         segment_ids, fetch)
    n = n_positions - start
    rows_var = np.asarray(rows_var, dtype=np.float32)
    if base is None:
        base = np.zeros((n, spec.n_heads, rows_var.shape[1]), dtype=np.float32)
    emb = base.copy()
    if idx_t:
        emb[np.array(idx_t), np.array(idx_h)] = rows_var[np.array(idx_r)]
    return emb.reshape(n, -1), (idx_t, idx_h, idx_r), nk, ni


def slot_keys(idx_t, idx_h, idx_r, n: int, n_heads: int) -> np.ndarray:
    """The variable of every slot ``t*H + h`` (``-1``: the table row)."""
    keys = np.full(n * n_heads, -1, dtype=np.int64)
    for t, h, r in zip(idx_t, idx_h, idx_r):
        keys[t * n_heads + h] = r
    return keys


def ple_true_emb(spec, tokens, t, fetch, overlay: dict | None = None) -> np.ndarray:
    """``Replica.ple_true_emb`` (``engraft/replica/model.py:473-495``):
    ``[1, H*D]`` f32, overlay rows replacing the matching global rows."""
    rows, data = row_set(spec, tokens, t, fetch)
    data = np.array(data, dtype=np.float32, copy=True)
    if overlay:
        for h in range(rows.shape[0]):
            g = int(rows[h])
            if g in overlay:
                data[h] = np.asarray(overlay[g], dtype=np.float32)
    return data.reshape(1, -1)
