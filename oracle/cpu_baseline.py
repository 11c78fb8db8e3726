"""Vectorized CPU restatement of the reference's table path, timed as
``bench.py``'s ``cpu_baseline`` (TEST INFRASTRUCTURE ONLY -- see
oracle/__init__.py).

This is the vectorized form of the reference's CPU path: the numpy-uint64 hash of
``engraft/damage.py:68-104`` (``oracle.hash.ngram_rows_np``), then
``torch.index_select`` gathers from a host-resident table of the benchmark's
full shape, Q8_0 dequantisation (``engraft/replica/dequant.py:86-93``), and an
fp32 add into the bf16 residual, on every host core torch uses.  The host table
is allocated at full size and only the rows the workload touches are written
(the rest stay untouched zero pages), so the gather walks the same 43.5 GB
address range as the device kernel.

``forward_q8_literal`` is the reference's path as written: one position at a
time, each re-hashing its whole prefix with the scalar hash
(``RowSet.from_position``, ``engraft/lens.py:126-136``, whose
``ngram_addresses(tokens[:t+1])`` makes the loop O(T^2)), one row read and
dequantisation per head, the concatenated rows added into that position's
residual row.

Pinned by tests/test_oracle_forward_backward.py (both forms bit-identical to
``oracle.forward.forward`` on the same inputs).
"""
from __future__ import annotations

import numpy as np
import torch

from oracle import formats as F
from oracle import hash as H
from oracle import synth


class HostTable:
    """Q8_0 split-layout table in host memory: int8 ``[n_rows, dim]`` and fp16
    ``[n_rows, dim/32]``, zero pages except for ``populate``d rows."""

    def __init__(self, n_rows: int, dim: int):
        self.n_rows = n_rows
        self.dim = dim
        self.payload = np.zeros((n_rows, dim), dtype=np.int8)
        self.scales = np.zeros((n_rows, dim // 32), dtype=np.float16)
        self.payload_t = torch.from_numpy(self.payload)
        self.scales_t = torch.from_numpy(self.scales)

    def populate(self, seed: int, rows, sigma: float = 0.02) -> int:
        uniq = np.unique(np.asarray(rows, dtype=np.int64).reshape(-1))
        for i in range(0, uniq.size, 1 << 16):
            part = uniq[i:i + (1 << 16)]
            q, d = synth.synth_rows("q8_0", seed, part, self.dim, sigma)
            self.payload[part] = q
            self.scales[part] = d
        return int(uniq.size)


def forward_q8(spec: H.HashSpec, tokens: np.ndarray, seq_len: int | None, table: HostTable,
               residual: torch.Tensor) -> tuple[np.ndarray, torch.Tensor]:
    """Hash -> gather -> dequant -> fp32 residual add -> bf16, on the CPU."""
    rows = H.ngram_rows_np(spec, tokens, seq_len=seq_len)
    p, hh = rows.shape
    idx = torch.from_numpy(rows.reshape(-1))
    q = torch.index_select(table.payload_t, 0, idx)
    d = torch.index_select(table.scales_t, 0, idx)
    nb = table.dim // 32
    emb = (q.view(p * hh, nb, 32).to(torch.float32) * d.to(torch.float32).unsqueeze(-1)).view(p, hh * table.dim)
    out = (residual.to(torch.float32) + emb).to(torch.bfloat16)
    return rows, out


def forward_literal(spec: H.HashSpec, tokens: np.ndarray, n_positions: int, read_row, dim: int,
                    residual: np.ndarray) -> np.ndarray:
    """``forward_q8_literal`` for any row format: ``read_row(r)`` returns global
    row ``r`` dequantised (f32 ``[dim]``), one call per head and position as the
    reference reads a row at a time."""
    toks = [int(x) for x in np.asarray(tokens[:n_positions])]
    out = np.empty((n_positions, spec.n_heads * dim), dtype=np.uint16)
    for t in range(n_positions):
        local = H.ngram_addresses_scalar(spec, toks[:t + 1])[t]
        emb = np.concatenate([read_row(H.local_to_global(spec, h, r)) for h, r in enumerate(local)])
        res = F.bf16_bits_to_f32(np.asarray(residual[t], dtype=np.uint16))
        out[t] = F.f32_to_bf16_bits((res + emb).astype(np.float32))
    return out


def forward_q8_literal(spec: H.HashSpec, tokens: np.ndarray, n_positions: int, table: HostTable,
                       residual: np.ndarray) -> np.ndarray:
    """The first ``n_positions`` positions of one sequence, position by position:
    the scalar hash of ``tokens[:t+1]`` (O(t) per position), the 16 global ids,
    a row read + Q8_0 dequantisation per head, fp32 add, RNE to bf16.  Returns
    the bf16 bit patterns ``uint16 [n_positions, n_heads * dim]``."""
    toks = [int(x) for x in np.asarray(tokens[:n_positions])]
    out = np.empty((n_positions, spec.n_heads * table.dim), dtype=np.uint16)
    for t in range(n_positions):
        local = H.ngram_addresses_scalar(spec, toks[:t + 1])[t]
        rows = [H.local_to_global(spec, h, r) for h, r in enumerate(local)]
        emb = np.concatenate([F.dequant_q8_0(table.payload[r:r + 1], table.scales[r:r + 1])[0] for r in rows])
        res = F.bf16_bits_to_f32(np.asarray(residual[t], dtype=np.uint16))
        out[t] = F.f32_to_bf16_bits((res + emb).astype(np.float32))
    return out
