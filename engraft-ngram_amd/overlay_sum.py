"""Overlay formats and merge on the device: the drop-ins for
``delta_for_pleo`` / ``sum_overlays`` (``engraft/replica/overlay_sum.py:
22-112``) and ``write_merged_pleo`` (``engraft/descend_corpus.py:627-647``).

``sum_overlays`` reads every ``.pleo`` file (host IO), then on the device:

* gathers the true rows of every file row and of the union (``eg_gather``);
* forms ``delta = rows_in_file - true_rows`` in fp32;
* sums the deltas of every union row over the files in file order, one
  fp32 addition at a time, as ``np.add.at`` does in the reference
  (``engraft/replica/overlay_sum.py:74-80``): ``eg_scatter_grad`` with one
  slot per file row keyed by the union's sorted ids adds a row's slots in slot
  order when no row has more than 32 of them; past that, each launch takes
  one layer of rows that are unique within it (a file's first occurrences,
  then its second ...), in file order, accumulating into the running sum;
* adds the sum to the union's true rows.

The manifest statistics (norms in float64, histograms) are computed on the
host from the device results, with the reference's formulas.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

from .descent import scatter_grad, true_rows_device as _true_rows_dev
from .lens import read_pleo, write_pleo

QUANT_FLOOR = 0.055  # engraft/replica/overlay_sum.py:19 (recorded only)
SEQUENTIAL_SLOTS = 32  # eg_scatter_grad adds at most this many slots of one row strictly in order


def _unique_layers(file_sizes: list[int], all_rows: np.ndarray) -> list[np.ndarray]:
    """Positions into the concatenated file rows, cut into layers whose rows
    are unique within the layer, in the order ``np.add.at`` visits them: per
    file, the first occurrence of each of its rows, then the second, ..."""
    layers = []
    start = 0
    for size in file_sizes:
        rows = all_rows[start:start + size]
        order = np.argsort(rows, kind="stable")
        srt = rows[order]
        head = np.ones(size, dtype=bool)
        head[1:] = srt[1:] != srt[:-1]
        run_start = np.flatnonzero(head)[np.cumsum(head) - 1] if size else np.empty(0, np.int64)
        occ = np.empty(size, dtype=np.int64)
        occ[order] = np.arange(size) - run_start
        for j in range(int(occ.max()) + 1 if size else 0):
            layers.append(start + np.flatnonzero(occ == j))
        start += size
    return layers


def delta_for_pleo(table, pleo_path) -> tuple[np.ndarray, np.ndarray]:
    """``(rows_global, delta)`` of one ``.pleo`` file, ``delta = rows_in_file -
    true_rows`` in fp32, in the file's row order
    (``engraft/replica/overlay_sum.py:22-35``)."""
    rows, data = read_pleo(pleo_path)
    true = _true_rows_dev(table, rows)
    delta = torch.as_tensor(data, device=table.device) - true
    return rows, delta.cpu().numpy()


def sum_overlays(table, pleo_paths: list) -> tuple[np.ndarray, np.ndarray, dict]:
    """``(rows_union, data_merged, manifest)`` over several ``.pleo`` files
    (``engraft/replica/overlay_sum.py:38-112``): ``rows_union`` int32 ascending,
    ``data_merged = true_rows(union) + sum_i delta_i`` (fp32), and the manifest
    with the reference's keys."""
    if not pleo_paths:
        raise ValueError("sum_overlays: no .pleo files provided")
    dev = table.device
    files = [read_pleo(p) for p in pleo_paths]
    row_len = files[0][1].shape[1]
    all_rows = np.concatenate([r for r, _ in files]).astype(np.int64)
    all_data = np.concatenate([d for _, d in files]).astype(np.float32)
    rows_union = np.unique(all_rows).astype(np.int32)
    n = rows_union.shape[0]

    # per file row: delta against the true row, on the device
    delta = torch.as_tensor(all_data, device=dev) - _true_rows_dev(table, all_rows)
    # sum over the files per union row, in file order
    ids = torch.as_tensor(rows_union, device=dev)
    idx = np.searchsorted(rows_union, all_rows)
    if n == 0 or int(np.bincount(idx, minlength=n).max()) <= SEQUENTIAL_SLOTS:
        delta_sum = scatter_grad(delta.contiguous(), torch.as_tensor(all_rows.astype(np.int32)).reshape(-1, 1),
                                 ids, row_len)
    else:
        delta_sum = torch.zeros((n, row_len), dtype=torch.float32, device=dev)
        for layer in _unique_layers([r.shape[0] for r, _ in files], all_rows):
            sel = torch.as_tensor(layer, device=dev)
            scatter_grad(delta.index_select(0, sel).contiguous(),
                         torch.as_tensor(all_rows[layer].astype(np.int32)).reshape(-1, 1), ids, row_len,
                         grad=delta_sum)
    true_union = _true_rows_dev(table, rows_union)
    data_merged = (true_union + delta_sum).cpu().numpy()

    # manifest (host, float64 norms as the reference)
    d_host = delta.cpu().numpy()
    row_norms = np.linalg.norm(d_host.astype(np.float64), axis=1)
    moved = row_norms > 0.0
    moved_count = np.zeros(n, dtype=np.int64)
    abs_sum = np.zeros(n, dtype=np.float64)
    np.add.at(moved_count, idx[moved], 1)
    np.add.at(abs_sum, idx[moved], row_norms[moved])
    sum_abs_norm = np.linalg.norm(delta_sum.cpu().numpy().astype(np.float64), axis=1)
    moved_any = moved_count >= 1
    shared = moved_count >= 2
    hist: dict[str, int] = {}
    for c in moved_count[moved_any].tolist():
        hist[str(int(c))] = hist.get(str(int(c)), 0) + 1
    sa, ab = sum_abs_norm[shared], abs_sum[shared]
    max_norm = float(sum_abs_norm.max()) if n else 0.0
    manifest = {
        "n_files": len(pleo_paths),
        "n_rows_union": int(n),
        "n_rows_moved_any": int(moved_any.sum()),
        "n_rows_shared": int(shared.sum()),
        "facts_per_row_histogram": hist,
        "shared_rows_sum_abs_norm_mean": float(sa.mean()) if sa.size else None,
        "shared_rows_sum_abs_norm_max": float(sa.max()) if sa.size else None,
        "shared_rows_abs_sum_norm_mean": float(ab.mean()) if ab.size else None,
        "shared_rows_abs_sum_norm_max": float(ab.max()) if ab.size else None,
        "max_row_delta_norm": max_norm,
        "quant_floor": QUANT_FLOOR,
        "max_row_delta_norm_over_quant_floor": max_norm > QUANT_FLOOR,
    }
    return rows_union, data_merged, manifest


def write_merged_pleo(table, row_map: dict, rows_var: torch.Tensor, all_read_rows, out_path: Path) -> dict:
    """``merged.pleo``: the variable rows (``row_map`` order, current values)
    then the other ``all_read_rows`` ascending at their true values
    (``engraft/descend_corpus.py:627-647``)."""
    variable = set(row_map.keys())
    frozen = sorted({int(r) for r in all_read_rows} - variable)
    rows_all = np.array(list(row_map.keys()) + frozen, dtype=np.int32)
    data_var = rows_var.detach().to("cpu", torch.float32).numpy()
    if frozen:
        data_frozen = _true_rows_dev(table, np.array(frozen, dtype=np.int64)).cpu().numpy()
        data_all = np.concatenate([data_var, data_frozen], axis=0) if data_var.shape[0] else data_frozen
    else:
        data_all = data_var
    write_pleo(out_path, rows_all, data_all)
    return {"n_rows_variable": len(row_map), "n_rows_frozen": len(frozen), "frozen_rows": frozen}
