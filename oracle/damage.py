"""Oracle: the damage plan's corpus scan (TEST INFRASTRUCTURE ONLY -- see
oracle/__init__.py).

``scan_hits`` restates ``engraft/damage.py:159-224`` step for step over
blocks with 2 tokens of history (``iter_blocks``, ``:107-118``), with the
vectorized hash of ``oracle.hash.ngram_rows_np`` in place of
``ngram_rows`` (``:68-104``).

Pinning (tests/test_oracle_overlay_emb.py): the reference's own known-answer test
``tests/test_damage.py:38-61`` (seed-7 FakeTable parameters, 20,000 tokens
with an EOS every 200, block 4,000: the hit positions equal those of the
scalar ``ngram_addresses`` loop, the last position never a hit), block-size
independence, and ``read_count`` against a brute-force count.
"""
from __future__ import annotations

import numpy as np

from oracle import hash as H


def iter_blocks(tokens, block: int, overlap: int = 2):
    n = len(tokens)
    offset = 0
    first = True
    while offset < n:
        this_block = min(block, n - offset)
        start = offset if first else offset - overlap
        yield offset, tokens[start:offset + this_block]
        offset += this_block
        first = False


def scan_hits(spec: H.HashSpec, tokens, overlay_sorted, dnorm_sorted, block: int) -> dict:
    tokens = np.asarray(tokens)
    n = int(tokens.shape[0])
    ov = np.asarray(overlay_sorted, dtype=np.int64)
    dnorm_sorted = np.asarray(dnorm_sorted, dtype=np.float32)
    n_ov = int(ov.shape[0])
    read_count = np.zeros(n_ov, dtype=np.int64)
    pos_parts, nh_parts, dmax_parts, dsum_parts = [], [], [], []
    hist = spec.ngram_size - 1
    for offset, blk in iter_blocks(tokens, block, hist):
        rows = H.ngram_rows_np(spec, blk)
        start_local = 0 if offset == 0 else hist
        rows = rows[start_local:]
        if rows.shape[0] == 0:
            continue
        idx = np.searchsorted(ov, rows)
        idx_c = np.clip(idx, 0, max(n_ov - 1, 0))
        matched = (n_ov > 0) & (idx < n_ov) & (ov[idx_c] == rows) if n_ov else np.zeros(rows.shape, bool)
        if not matched.any():
            continue
        np.add.at(read_count, idx_c[matched], 1)
        md = np.where(matched, dnorm_sorted[idx_c], np.float32(0.0)).astype(np.float32)
        n_hit = matched.sum(axis=1)
        hit_local = np.flatnonzero(n_hit > 0)
        pos_here = (offset + hit_local).astype(np.int64)
        keep = pos_here < (n - 1)
        hit_local, pos_here = hit_local[keep], pos_here[keep]
        if hit_local.size:
            pos_parts.append(pos_here)
            nh_parts.append(n_hit[hit_local].astype(np.int32))
            dmax_parts.append(md[hit_local].max(axis=1).astype(np.float32))
            dsum_parts.append(md[hit_local].sum(axis=1, dtype=np.float64).astype(np.float32))

    def _cat(parts, dtype):
        return np.concatenate(parts) if parts else np.zeros(0, dtype=dtype)

    return {"pos": _cat(pos_parts, np.int64), "n_hit_rows": _cat(nh_parts, np.int32),
            "dnorm_max": _cat(dmax_parts, np.float32), "dnorm_sum": _cat(dsum_parts, np.float32),
            "read_count": read_count, "n_tokens": n}
