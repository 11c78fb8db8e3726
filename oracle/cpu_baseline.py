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
``oracle.forward.forward`` on the same inputs) and tests/test_cpu_baselines.py
(``scan_block_threads`` equal to ``oracle.damage.scan_hits``; ``TorchDescent``
within 1e-5 of the oracle's scatter + Adam, its requantisation equal to
``oracle.formats.quant_q8_0``).
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


# ---------------------------------------------------------------------------
# Descent step and damage scan on every host thread
# ---------------------------------------------------------------------------
class TorchDescent:
    """The descent step as the reference's CPU torch path would run it on the
    full config-2 inputs (``engraft/replica/seq.py:433-441`` autograd of the
    ``index_put``, i.e. an ``index_add_`` over the slots; ``torch.optim.Adam``
    of ``engraft/descend_corpus.py:785-790, 921-947``), then the Q8_0
    requantisation of the updated rows, on every thread torch uses.

    ``rows`` int ``[P, H]`` global ids; ``param0`` f32 ``[U, dim]`` the true rows
    of the sorted unique ids; ``lr`` as the GPU leg."""

    def __init__(self, rows: torch.Tensor, param0: torch.Tensor, lr: float):
        flat = rows.reshape(-1).to(torch.int64)
        self.ids, self.inv = torch.unique(flat, sorted=True, return_inverse=True)
        self.dim = int(param0.shape[1])
        self.param = param0.clone().requires_grad_(True)
        self.opt = torch.optim.Adam([self.param], lr=lr)

    def step(self, d_res: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        d = d_res.to(torch.float32).reshape(-1, self.dim)
        grad = torch.zeros_like(self.param, requires_grad=False)
        grad.index_add_(0, self.inv, d)
        self.param.grad = grad
        self.opt.step()
        with torch.no_grad():
            blocks = self.param.detach().reshape(-1, self.dim // 32, 32)
            dq = (blocks.abs().amax(dim=-1) / 127.0).to(torch.float16)
            d32 = dq.to(torch.float32).unsqueeze(-1)
            q = torch.where(d32 == 0, torch.zeros_like(blocks), torch.round(blocks / d32))
            q = q.clamp_(-127, 127).to(torch.int8)
        return q.reshape(-1, self.dim), dq


def _scan_chunk(spec: H.HashSpec, tokens: np.ndarray, lo: int, hi: int, ov: np.ndarray, dnorm: np.ndarray):
    """Positions [lo, hi) of one block (the block is one sequence): hits per
    position, their dnorm max and sum, and the overlay indices hit."""
    hist = spec.ngram_size - 1
    s0 = max(0, lo - hist)
    rows = H.ngram_rows_np(spec, tokens[s0:hi])[lo - s0:]
    idx = np.searchsorted(ov, rows)
    idx_c = np.minimum(idx, ov.size - 1)
    matched = ov[idx_c] == rows
    md = np.where(matched, dnorm[idx_c], np.float32(0.0)).astype(np.float32)
    n_hit = matched.sum(axis=1).astype(np.int32)
    dmax = np.where(n_hit > 0, md.max(axis=1), np.float32(0.0)).astype(np.float32)
    dsum = md.sum(axis=1, dtype=np.float64).astype(np.float32)
    return n_hit, dmax, dsum, idx_c[matched]


def scan_block_threads(spec: H.HashSpec, tokens, ov_sorted, dnorm_sorted, threads: int, pool=None) -> dict:
    """The damage scan of one token block (``engraft/damage.py:168-224``:
    vectorized numpy-uint64 hash, ``searchsorted`` membership, per-position
    count / max / sum, read counts) split into ``threads`` chunks run on a
    thread pool (numpy releases the GIL inside its array operations).  Returns
    every position's ``n_hit``, ``dnorm_max``, ``dnorm_sum`` and the overlay
    rows' ``read_count``."""
    from concurrent.futures import ThreadPoolExecutor

    tokens = np.asarray(tokens)
    ov = np.asarray(ov_sorted, dtype=np.int64)
    dn = np.asarray(dnorm_sorted, dtype=np.float32)
    n = tokens.shape[0]
    bounds = np.linspace(0, n, threads + 1).astype(np.int64)
    own = pool is None
    pool = pool or ThreadPoolExecutor(threads)
    try:
        parts = list(pool.map(lambda i: _scan_chunk(spec, tokens, int(bounds[i]), int(bounds[i + 1]), ov, dn),
                              range(threads)))
    finally:
        if own:
            pool.shutdown()
    read_count = np.zeros(ov.size, dtype=np.int64)
    for p in parts:
        read_count += np.bincount(p[3], minlength=ov.size)
    return {"n_hit": np.concatenate([p[0] for p in parts]), "dnorm_max": np.concatenate([p[1] for p in parts]),
            "dnorm_sum": np.concatenate([p[2] for p in parts]), "read_count": read_count}
