"""Packing of fragments into fixed-length bins: the drop-in for
``engraft/replica/pack.py:60-161`` (data only; host logic).

Each fragment becomes ``[eos] + frag``; bins fill greedily in order; a
fragment longer than ``max_len`` on its own raises ``ValueError``.  A packed
sequence's ``segment_ids`` / ``positions`` cover its ``len(tokens) - 1`` prefix
positions, and ``seg_start`` gives every position the index of its segment's
first token -- the segment start the device hash never looks before
(``engraft/replica/seq.py:392-399``).
"""
from __future__ import annotations

import dataclasses

import numpy as np
import torch


@dataclasses.dataclass
class Packed:
    """One greedily-filled bin (``engraft/replica/pack.py:60-96``)."""

    tokens: list[int]
    segment_ids: torch.Tensor  # [n_prefix] int64
    positions: torch.Tensor  # [n_prefix] float64
    frag_slices: list[tuple[int, int]]

    def to(self, device) -> "Packed":
        return Packed(tokens=self.tokens, segment_ids=self.segment_ids.to(device),
                      positions=self.positions.to(device), frag_slices=self.frag_slices)

    def seg_start(self) -> np.ndarray:
        """int32 ``[n_prefix]``: the first index of each position's segment."""
        return seg_starts_from_segment_ids(self.segment_ids)


def seg_starts_from_segment_ids(segment_ids) -> np.ndarray:
    """First index of every position's segment, from contiguous increasing
    ``segment_ids`` (``engraft/replica/seq.py:299-322``)."""
    seg = segment_ids.detach().to("cpu").numpy() if isinstance(segment_ids, torch.Tensor) \
        else np.asarray(segment_ids)
    n = seg.shape[0]
    if n == 0:
        return np.zeros(0, dtype=np.int32)
    change = np.ones(n, dtype=bool)
    change[1:] = seg[1:] != seg[:-1]
    starts = np.flatnonzero(change)
    return starts[np.cumsum(change) - 1].astype(np.int32)


def _bin_ranges(lengths: np.ndarray, max_len: int) -> list[tuple[int, int]]:
    """``[first, end)`` fragment ranges of the bins.  A bin keeps taking the
    next fragment while the total canonical length stays within ``max_len``;
    the first fragment that does not fit opens the next bin (no reordering)."""
    ranges: list[tuple[int, int]] = []
    first, used = 0, 0
    for i, ln in enumerate(lengths.tolist()):
        if i > first and used + ln > max_len:
            ranges.append((first, i))
            first, used = i, 0
        used += ln
    if lengths.size > first:
        ranges.append((first, int(lengths.size)))
    return ranges


def pack_fragments(frags: list[list[int]], eos: int, max_len: int) -> list[Packed]:
    """Greedy in-order packing of ``[eos] + frag`` fragments into bins of at
    most ``max_len`` tokens (``engraft/replica/pack.py:99-161``).

    Per bin, fragment k occupies tokens ``[off_k, off_k + len_k)``; every prefix
    position (``len(tokens) - 1`` of them) carries its fragment index and its
    offset inside the fragment, and ``frag_slices[k] = (off_k, off_k + len_k - 1)``
    leaves out the fragment's last position (the boundary, or the bin's final
    label).  ``ValueError`` when one fragment alone exceeds ``max_len``."""
    lengths = np.fromiter((len(f) + 1 for f in frags), dtype=np.int64, count=len(frags))
    too_long = np.flatnonzero(lengths > max_len)
    if too_long.size:
        i = int(too_long[0])
        raise ValueError(f"pack_fragments: fragment {i} (canonical length {int(lengths[i])}, with EOS) "
                         f"exceeds max_len={max_len} on its own")
    out: list[Packed] = []
    for first, end in _bin_ranges(lengths, max_len):
        lens = lengths[first:end]
        offs = np.cumsum(lens) - lens
        total = int(lens.sum())
        n_prefix = total - 1
        tokens: list[int] = []
        for f in frags[first:end]:
            tokens.append(eos)
            tokens.extend(f)
        local = np.arange(end - first, dtype=np.int64)
        seg = np.repeat(local, lens)[:n_prefix]
        pos = (np.arange(total, dtype=np.int64) - np.repeat(offs, lens))[:n_prefix]
        out.append(Packed(tokens=tokens, segment_ids=torch.from_numpy(seg.copy()),
                          positions=torch.from_numpy(pos.astype(np.float64)),
                          frag_slices=[(int(o), int(o + ln - 1)) for o, ln in zip(offs, lens)]))
    return out
