"""Overlay rows resolved per global id on the device: the drop-in for the
reference's overlay substitution (``Replica.ple_true_emb(tokens, t, overlay)``,
``engraft/replica/model.py:473-495``; the int-key branch of
``OverlayEmb.build``, ``engraft/replica/seq.py:412-441``; the engine's
``.pleo`` substitution at gather time).

``DeviceOverlay`` holds a sorted, unique int32 id array plus the replacement
rows (fp32 as in ``.pleo`` files, or block-quantised like the base table) in
HBM; the forward kernels binary-search every slot's row id in it and read the
replacement instead of the base row.  ``with_bitmap(n_rows)`` adds the
two-level rank bitmap of the ids (``eg_build_id_bitmap``, about n_rows / 4
bytes), with which a lookup costs one or two probes instead of the search.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _lib
from .table import RowStore


def _device(device) -> torch.device:
    if device is None:
        return torch.device("cuda", torch.cuda.current_device())
    return torch.device(device)


class DeviceOverlay:
    """Sorted unique global row ids -> replacement rows, resident in HBM.

    ``index`` (optional, int32 ``[n]``): row of ``rows`` holding the k-th id;
    without it the k-th id reads row k."""

    def __init__(self, ids: torch.Tensor, rows: RowStore, index: torch.Tensor | None = None, *,
                 ids_checked: bool = False):
        if ids.dtype != torch.int32 or ids.dim() != 1 or not ids.is_contiguous():
            raise ValueError("overlay ids must be a contiguous 1-D int32 tensor")
        # Both lookups (binary search, rank bitmap) need strictly ascending ids;
        # ids_checked: the caller has already established that.
        if not ids_checked and ids.numel() > 1 and not bool((ids[1:] > ids[:-1]).all()):
            raise ValueError("overlay ids must be sorted ascending and unique")
        if ids.numel() and not ids_checked and int(ids[0]) < 0:
            raise ValueError("overlay ids must be global rows >= 0")
        if index is None and rows.n_rows < ids.numel():
            raise ValueError(f"{ids.numel()} overlay ids but only {rows.n_rows} rows")
        if index is not None and (index.dtype != torch.int32 or index.shape != ids.shape):
            raise ValueError("overlay index must be int32 with the shape of ids")
        self.ids = ids
        self.rows = rows
        self.index = index
        self.bitmap = None
        self.n_bits = 0

    def with_bitmap(self, n_rows: int) -> "DeviceOverlay":
        """Builds the rank bitmap of the ids over ``n_rows`` global rows (every
        row id the table can produce: its ``n_rows``) and returns self; lookups
        then resolve through it, with the same results."""
        n_rows = int(n_rows)
        if not 1 <= n_rows <= (1 << 31):
            raise ValueError(f"n_rows={n_rows} out of range")
        if self.n and int(self.ids[-1]) >= n_rows:
            # the bitmap holds rows below n_rows only: a larger id would be
            # found by the binary search and missed through the bitmap
            raise ValueError(f"overlay id {int(self.ids[-1])} >= n_rows={n_rows}")
        bm = torch.empty(int(_lib.load().eg_id_bitmap_words(n_rows)), dtype=torch.int32, device=self.ids.device)
        _lib.call("eg_build_id_bitmap", _lib.ptr(self.ids), self.n, _lib.ptr(bm), n_rows,
                  _lib.stream_ptr(self.ids.device))
        self.bitmap, self.n_bits = bm, n_rows
        return self

    @property
    def n(self) -> int:
        return int(self.ids.numel())

    def __len__(self) -> int:
        return self.n

    def c_overlay(self) -> _lib.EgOverlay:
        o = _lib.EgOverlay()
        o.n = self.n
        o.ids = _lib.ptr(self.ids)
        o.index = _lib.ptr(self.index)
        o.rows = self.rows.c_table()
        o.bitmap = _lib.ptr(self.bitmap)
        o.n_bits = self.n_bits
        return o

    # ---- construction ----------------------------------------------------------------------
    @staticmethod
    def _sorted_ids(ids) -> tuple[np.ndarray, np.ndarray]:
        ids = np.asarray(ids, dtype=np.int64).reshape(-1)
        if ids.size and (ids.min() < 0 or ids.max() > np.iinfo(np.int32).max):
            raise ValueError("overlay ids must be global rows in [0, 2^31)")
        order = np.argsort(ids, kind="stable")
        s = ids[order]
        if s.size > 1 and np.any(s[1:] == s[:-1]):
            dup = int(s[1:][s[1:] == s[:-1]][0])
            raise ValueError(f"global row {dup} appears twice in the overlay")
        return s.astype(np.int32), order

    @classmethod
    def from_rows(cls, ids, data, device=None) -> "DeviceOverlay":
        """fp32 replacement vectors ``data [n, D]`` for global ``ids [n]``
        (the ``.pleo`` / ``{global_row: vector}`` form)."""
        dev = _device(device)
        data = np.asarray(data, dtype=np.float32)
        s, order = cls._sorted_ids(ids)
        if data.ndim != 2 or data.shape[0] != s.size:
            raise ValueError(f"data must be [n, D] with n={s.size}")
        payload = torch.from_numpy(np.ascontiguousarray(data[order])).to(dev)
        return cls(torch.from_numpy(s).to(dev), RowStore("f32", data.shape[1], payload), ids_checked=True)

    @classmethod
    def from_dict(cls, overlay: dict, dim: int, device=None) -> "DeviceOverlay":
        """``{global_row: vector[dim]}`` (``engraft/replica/model.py:473-495``)."""
        if not overlay:
            return cls.from_rows(np.zeros(0, dtype=np.int64), np.zeros((0, dim), np.float32), device)
        keys = list(overlay.keys())
        data = np.stack([np.asarray(overlay[k], dtype=np.float32).reshape(dim) for k in keys])
        return cls.from_rows(np.array(keys, dtype=np.int64), data, device)

    @classmethod
    def from_quantized(cls, fmt: str, ids, payload, scales=None, device=None) -> "DeviceOverlay":
        """Replacement rows already in a block format (``payload``/``scales`` as
        numpy arrays in the split layout of ``fmt``)."""
        dev = _device(device)
        s, order = cls._sorted_ids(ids)
        payload = np.ascontiguousarray(np.asarray(payload)[order])
        n = s.size
        from .table import payload_shape, scales_shape

        if fmt == "q8_0" or fmt == "mxfp8":
            dim = payload.shape[1]
        elif fmt == "bf16":
            dim = payload.shape[1]
        else:
            raise ValueError(f"from_quantized: unsupported format {fmt!r}")
        shp, dt = payload_shape(fmt, n, dim)
        p = torch.from_numpy(payload.view(np.uint8).reshape(n, -1)).view(dt).reshape(shp).to(dev)
        st = None
        ss = scales_shape(fmt, n, dim)
        if ss is not None:
            sc = np.ascontiguousarray(np.asarray(scales)[order])
            st = torch.from_numpy(sc.view(np.uint8).reshape(n, -1)).view(ss[1]).reshape(ss[0]).to(dev)
        return cls(torch.from_numpy(s).to(dev), RowStore(fmt, dim, p, st), ids_checked=True)

    @classmethod
    def from_store(cls, ids: torch.Tensor, rows: RowStore, index: torch.Tensor | None = None) -> "DeviceOverlay":
        """Device-resident ids (sorted, unique) over an existing row store."""
        return cls(ids.to(torch.int32).contiguous(), rows, index)
