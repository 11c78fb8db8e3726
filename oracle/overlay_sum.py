"""Oracle: the merge of several overlays (TEST INFRASTRUCTURE ONLY -- see
oracle/__init__.py).

``sum_overlays`` restates ``engraft/replica/overlay_sum.py:38-112`` with the
true rows supplied by ``fetch(ids)``: ``delta_i = rows_i - true`` in fp32, the
union of the files' rows ascending, ``np.add.at`` of each file's deltas into
one fp32 running sum, file after file (``engraft/replica/overlay_sum.py:74-80``:
one addition at a time, in file order, for any number of files), and
``merged = true_union + delta_sum``.  ``write_merged_rows`` restates the row
order of ``engraft/descend_corpus.py:627-647``.

Pinning (tests/test_oracle_overlay_emb.py): against a per-row dictionary loop
(brute force), the single-file identity ``merged == true + (data - true)``,
an untouched row's exact-zero delta, and the manifest counts on a hand-built
three-file case.
"""
from __future__ import annotations

import numpy as np


def sum_overlays(files: list[tuple[np.ndarray, np.ndarray]], fetch) -> tuple[np.ndarray, np.ndarray, dict]:
    rows_union = np.array(sorted({int(r) for rows, _ in files for r in rows.tolist()}), dtype=np.int32)
    row_index = {int(g): i for i, g in enumerate(rows_union)}
    n = rows_union.shape[0]
    row_len = files[0][1].shape[1]
    per_file = []
    for rows, data in files:
        per_file.append((rows, (np.asarray(data, np.float32) - fetch(rows).astype(np.float32)).astype(np.float32)))
    # delta sum per union row: file after file, np.add.at (sequential fp32)
    delta_sum = np.zeros((n, row_len), dtype=np.float32)
    for rows, delta in per_file:
        np.add.at(delta_sum, np.array([row_index[int(g)] for g in rows.tolist()], dtype=np.int64), delta)
    moved_count = np.zeros(n, dtype=np.int64)
    abs_sum = np.zeros(n, dtype=np.float64)
    for rows, delta in per_file:
        norms = np.linalg.norm(delta.astype(np.float64), axis=1)
        m = norms > 0.0
        idx = np.array([row_index[int(g)] for g in rows.tolist()], dtype=np.int64)
        np.add.at(moved_count, idx[m], 1)
        np.add.at(abs_sum, idx[m], norms[m])
    merged = (fetch(rows_union).astype(np.float32) + delta_sum).astype(np.float32)
    sum_abs = np.linalg.norm(delta_sum.astype(np.float64), axis=1)
    hist: dict[str, int] = {}
    for c in moved_count[moved_count >= 1].tolist():
        hist[str(int(c))] = hist.get(str(int(c)), 0) + 1
    shared = moved_count >= 2
    manifest = {"n_files": len(files), "n_rows_union": int(n), "n_rows_moved_any": int((moved_count >= 1).sum()),
                "n_rows_shared": int(shared.sum()), "facts_per_row_histogram": hist,
                "shared_rows_sum_abs_norm_max": float(sum_abs[shared].max()) if shared.any() else None,
                "shared_rows_abs_sum_norm_max": float(abs_sum[shared].max()) if shared.any() else None,
                "max_row_delta_norm": float(sum_abs.max()) if n else 0.0}
    return rows_union, merged, manifest


def write_merged_rows(row_map: dict, rows_var: np.ndarray, all_read_rows, fetch):
    """Rows and data of ``merged.pleo``: variables in ``row_map`` order, then
    the frozen rows ascending at their true values."""
    frozen = sorted({int(r) for r in all_read_rows} - set(row_map.keys()))
    rows = np.array(list(row_map.keys()) + frozen, dtype=np.int32)
    data = np.asarray(rows_var, np.float32)
    if frozen:
        data = np.concatenate([data, fetch(np.array(frozen)).astype(np.float32)]) if data.shape[0] else \
            fetch(np.array(frozen)).astype(np.float32)
    return rows, data
