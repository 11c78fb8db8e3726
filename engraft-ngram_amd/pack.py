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


def pack_fragments(frags: list[list[int]], eos: int, max_len: int) -> list[Packed]:
    """``engraft/replica/pack.py:99-161``: greedy, in order, no reordering."""
    canon = [[eos] + list(f) for f in frags]
    lengths = [len(c) for c in canon]
    for i, ln in enumerate(lengths):
        if ln > max_len:
            raise ValueError(f"pack_fragments: fragment {i} (canonical length {ln}, with EOS) "
                             f"exceeds max_len={max_len} on its own")
    bins: list[list[int]] = []
    cur: list[int] = []
    cur_len = 0
    for i, ln in enumerate(lengths):
        if cur and cur_len + ln > max_len:
            bins.append(cur)
            cur, cur_len = [], 0
        cur.append(i)
        cur_len += ln
    if cur:
        bins.append(cur)
    out: list[Packed] = []
    for bin_idxs in bins:
        tok_offsets: list[int] = []
        tokens: list[int] = []
        for fi in bin_idxs:
            tok_offsets.append(len(tokens))
            tokens.extend(canon[fi])
        n_prefix = len(tokens) - 1
        seg = torch.zeros(n_prefix, dtype=torch.int64)
        pos = torch.zeros(n_prefix, dtype=torch.float64)
        frag_slices: list[tuple[int, int]] = []
        for local_seg, fi in enumerate(bin_idxs):
            off, ln = tok_offsets[local_seg], lengths[fi]
            end_all = min(off + ln, n_prefix)
            if end_all > off:
                seg[off:end_all] = local_seg
                pos[off:end_all] = torch.arange(end_all - off, dtype=torch.float64)
            frag_slices.append((off, off + ln - 1))
        out.append(Packed(tokens=tokens, segment_ids=seg, positions=pos, frag_slices=frag_slices))
    return out
