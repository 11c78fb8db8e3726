"""The lens, device edition: the drop-in for the table-path half of
``engraft.lens`` (``engraft/lens.py:25-198``).

* ``write_pleo`` / ``read_pleo`` -- the ``.pleo`` overlay format, byte for byte
  (``b"PLEO"``, ``<u32 n>``, ``<u32 dim>``, ``<i4 rows[n]>``, ``<f4 data[n*dim]>``;
  ``engraft/lens.py:33-59``).  Host file IO; ``pleo_overlay`` turns a file into a
  ``DeviceOverlay`` the forward kernels resolve per id.
* ``local_to_global`` (``engraft/lens.py:108-110``).
* ``RowSet`` -- the ``n_heads`` rows of one position with their global ids
  (``engraft/lens.py:118-198``): the hash and the gather run on the device,
  ``rows_global``/``data`` come back as host arrays like the reference's, and the
  variant generators and ``build_overlay`` keep the reference's semantics.

The ``.pleo`` dimension is the table's row length (160 for the reference's real
tables; the synthetic tables of BASELINE use 128).
"""
from __future__ import annotations

import dataclasses
import struct
from pathlib import Path

import numpy as np

from .overlay import DeviceOverlay

PLEO_MAGIC = b"PLEO"


def write_pleo(path: str | Path, rows_global, data, dim: int | None = None) -> None:
    """Writes a .pleo file: magic PLEO, uint32 n, uint32 dim, int32 rows[n],
    f32 data[n*dim] (``engraft/lens.py:33-46``; same ``ValueError``s)."""
    rows = np.asarray(rows_global, dtype="<i4")
    values = np.asarray(data, dtype="<f4")
    n = rows.shape[0]
    d = values.shape[1] if (dim is None and values.ndim == 2) else dim
    if d is None or values.shape != (n, d):
        raise ValueError(f"data.shape={values.shape}, expected ({n}, {d})")
    if rows.ndim != 1:
        raise ValueError(f"rows_global must be 1-D, got ndim={rows.ndim}")
    with open(path, "wb") as f:
        f.write(PLEO_MAGIC)
        f.write(struct.pack("<II", n, d))
        f.write(rows.tobytes())
        f.write(values.tobytes())


def read_pleo(path: str | Path) -> tuple[np.ndarray, np.ndarray]:
    """Reads a .pleo file: ``(rows_global int32 [n], data float32 [n, dim])``
    (``engraft/lens.py:49-59``; ``ValueError`` on a bad magic)."""
    with open(path, "rb") as f:
        magic = f.read(4)
        if magic != PLEO_MAGIC:
            raise ValueError(f"bad magic: {magic!r}, expected {PLEO_MAGIC!r}")
        n, dim = struct.unpack("<II", f.read(8))
        rows = np.frombuffer(f.read(n * 4), dtype="<i4").astype(np.int32).copy()
        data = np.frombuffer(f.read(n * dim * 4), dtype="<f4").astype(np.float32).copy()
        data = data.reshape(n, dim)
    return rows, data


def pleo_overlay(path: str | Path, device=None) -> DeviceOverlay:
    """A ``.pleo`` file as a device overlay (the engine's gather-time
    substitution, ``engine/README.md:8-16``): rows sorted by id in HBM."""
    rows, data = read_pleo(path)
    return DeviceOverlay.from_rows(rows, data, device=device)


def local_to_global(table, h: int, row_local: int) -> int:
    """Global row index in the merged layout (local + head_offsets[h])."""
    return int(table.head_offsets[h]) + int(row_local)


@dataclasses.dataclass
class RowSet:
    """The ``n_heads`` true rows read at a position, with their global ids
    (``engraft/lens.py:118-165``)."""

    table: object
    rows_global: np.ndarray  # int32 [n_heads]
    data: np.ndarray  # float32 [n_heads, row_len]

    @classmethod
    def from_position(cls, table, tokens: list[int], t: int) -> "RowSet":
        """The RowSet of position ``t`` of ``tokens``: hash + gather on the device.
        Position t's context is tokens ``t-ngram_size+1 .. t``, so only that window
        is hashed (the reference re-hashes the whole prefix per call,
        ``engraft/lens.py:129``)."""
        if not 0 <= t < len(tokens):
            raise IndexError(f"position {t} outside [0, {len(tokens)})")
        window = list(tokens[max(0, t - table.ngram_size + 1):t + 1])
        rows = table.rows(window).cpu().numpy()[-1].astype(np.int32)
        data = table.gather(table_rows_tensor(table, rows)).cpu().numpy().reshape(table.n_heads, table.row_len)
        return cls(table=table, rows_global=rows, data=data)

    # -- variants: each returns a new float32 array [n_heads, row_len] --
    def identity(self) -> np.ndarray:
        return self.data.copy()

    def zero(self) -> np.ndarray:
        return np.zeros_like(self.data)

    def scale(self, k: float) -> np.ndarray:
        return (self.data * k).astype(np.float32)

    def random_matched(self, rng: np.random.Generator) -> np.ndarray:
        """Independent Gaussian per row, renormalised to the true row's norm."""
        norms = np.linalg.norm(self.data, axis=1, keepdims=True)
        g = rng.standard_normal(self.data.shape).astype(np.float32)
        g_norms = np.linalg.norm(g, axis=1, keepdims=True)
        g_norms = np.where(g_norms == 0.0, 1.0, g_norms)
        return (g / g_norms * norms).astype(np.float32)

    def swap(self, other: "RowSet") -> np.ndarray:
        if other.data.shape != self.data.shape:
            raise ValueError("swap: RowSet of different shape")
        return other.data.copy()

    def isolate(self, h: int) -> np.ndarray:
        out = np.zeros_like(self.data)
        out[h] = self.data[h]
        return out

    @staticmethod
    def build_overlay(parts: list[tuple[np.ndarray, np.ndarray]]) -> tuple[np.ndarray, np.ndarray]:
        """Merges several ``(rows_global, data[n, D])`` sets by global row,
        deduplicating; ``ValueError`` if one row receives two different vectors
        (``engraft/lens.py:167-198``).  Returns ascending rows."""
        seen: dict[int, np.ndarray] = {}
        dim = None
        for rows_global, data in parts:
            rows_global = np.asarray(rows_global)
            data = np.asarray(data, dtype=np.float32)
            if rows_global.shape[0] != data.shape[0]:
                raise ValueError("build_overlay: rows_global and data of different length")
            if data.ndim == 2:
                dim = data.shape[1]
            for i in range(rows_global.shape[0]):
                r = int(rows_global[i])
                vec = data[i]
                if r in seen:
                    if not np.array_equal(seen[r], vec):
                        raise ValueError(f"build_overlay: global row {r} receives two different vectors")
                else:
                    seen[r] = vec
        if not seen:
            return np.empty(0, dtype=np.int32), np.empty((0, dim or 0), dtype=np.float32)
        rows_sorted = sorted(seen.keys())
        return np.array(rows_sorted, dtype=np.int32), np.stack([seen[r] for r in rows_sorted]).astype(np.float32)


def table_rows_tensor(table, rows: np.ndarray):
    import torch

    return torch.as_tensor(np.asarray(rows, dtype=np.int32).reshape(-1, 1), device=table.device)
