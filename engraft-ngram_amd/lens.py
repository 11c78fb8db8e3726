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
tables; the benchmark's synthetic tables use 128).
"""
from __future__ import annotations

import dataclasses
import struct
from pathlib import Path

import numpy as np

from .overlay import DeviceOverlay
from .table import ROW_LEN

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

    # -- variants of the true rows (engraft/lens.py:138-165): each a new float32
    #    array of the same [n_heads, row_len] shape --
    def identity(self) -> np.ndarray:
        return np.array(self.data, dtype=np.float32, copy=True)

    def zero(self) -> np.ndarray:
        return np.zeros(self.data.shape, dtype=np.float32)

    def scale(self, k: float) -> np.ndarray:
        return np.multiply(self.data, np.float32(k), dtype=np.float32)

    def random_matched(self, rng: np.random.Generator) -> np.ndarray:
        """Gaussian rows with the true rows' norms.  One ``standard_normal`` draw
        of the whole [n_heads, row_len] block, so the same generator state gives
        the reference's numbers; an all-zero draw row keeps norm 1."""
        target = np.linalg.norm(self.data, axis=1, keepdims=True)
        draw = rng.standard_normal(self.data.shape).astype(np.float32)
        drawn = np.linalg.norm(draw, axis=1, keepdims=True)
        drawn = drawn + (drawn == 0.0)  # 0 -> 1, every other norm unchanged
        return ((draw / drawn) * target).astype(np.float32)

    def swap(self, other: "RowSet") -> np.ndarray:
        """The other position's rows in place of these (shapes must agree)."""
        if other.data.shape != self.data.shape:
            raise ValueError("swap: RowSet of different shape")
        return np.array(other.data, dtype=np.float32, copy=True)

    def isolate(self, h: int) -> np.ndarray:
        """Head ``h``'s row kept, every other head zeroed (negative ``h`` counts
        from the end, like an index)."""
        keep = range(self.data.shape[0])[h]
        mask = (np.arange(self.data.shape[0]) == keep)[:, None]
        return np.where(mask, self.data, np.float32(0.0)).astype(np.float32)

    @staticmethod
    def build_overlay(parts: list[tuple[np.ndarray, np.ndarray]]) -> tuple[np.ndarray, np.ndarray]:
        """One overlay from several ``(rows_global, data[n, D])`` sets
        (``engraft/lens.py:167-198``): rows ascending, each once.  A row listed
        more than once must carry equal vectors every time (``ValueError``
        otherwise: NaN never equals itself, -0.0 equals 0.0).

        All parts are concatenated and stably sorted by row; every later member
        of a run of equal rows is compared against the run's first member, which
        is kept.  A first member is never compared with itself, so a row seen
        once is accepted whatever it holds (NaN included)."""
        rows_parts, data_parts = [], []
        dim = None
        for rows_global, data in parts:
            r = np.asarray(rows_global).reshape(-1)
            d = np.asarray(data, dtype=np.float32)
            if r.shape[0] != d.shape[0]:
                raise ValueError("build_overlay: rows_global and data of different length")
            if d.ndim == 2:
                dim = d.shape[1]
            rows_parts.append(r.astype(np.int64))
            data_parts.append(d.reshape(d.shape[0], -1))
        n = sum(r.shape[0] for r in rows_parts)
        if n == 0:
            return np.empty(0, dtype=np.int32), np.empty((0, ROW_LEN if dim is None else dim), dtype=np.float32)
        rows = np.concatenate(rows_parts)
        data = np.concatenate(data_parts, axis=0)
        order = np.argsort(rows, kind="stable")
        rows, data = rows[order], data[order]
        head = np.ones(n, dtype=bool)
        head[1:] = rows[1:] != rows[:-1]
        first = np.flatnonzero(head)[np.cumsum(head) - 1]  # each entry's run head
        clash = ~head & ~(data == data[first]).all(axis=1)
        if clash.any():
            raise ValueError(f"build_overlay: global row {int(rows[np.flatnonzero(clash)[0]])} "
                             "receives two different vectors")
        return rows[head].astype(np.int32), np.ascontiguousarray(data[head])


def table_rows_tensor(table, rows: np.ndarray):
    import torch

    return torch.as_tensor(np.asarray(rows, dtype=np.int32).reshape(-1, 1), device=table.device)
