"""The damage plan's table half on the device: the drop-in for
``ngram_rows`` / ``iter_blocks`` / ``scan_hits`` / ``compute_rows_delta``
(``engraft/damage.py:68-224``).

``scan_hits`` runs one fused launch per corpus block (``eg_scan_overlay``):
every position hashes its ``n_heads`` rows (the whole block as one sequence,
so every position sees its real predecessors), looks each up in the sorted
overlay ids, counts the reads of every overlay row and reduces per position
the number of overlay rows read and the max / sum of their ``dnorm``.  Blocks
overlap by ``ngram_size - 1`` tokens, whose positions are dropped, so the
result equals a scan of the whole corpus as one sequence.
"""
from __future__ import annotations

import ctypes
import time
from typing import Iterator

import numpy as np
import torch

from . import _lib
from .descent import _read_true_rows

BLOCK_TOKENS = 8_000_000  # engraft/damage.py:60


def ngram_rows(tokens: np.ndarray, table) -> tuple[np.ndarray, ...]:
    """Global rows of every position of ``tokens``, one int64 ``[n,
    heads_per_ngram]`` array per n-gram order (bigram, trigram, ...;
    ``engraft/damage.py:68-104`` returns the bigram and trigram arrays of an
    ``ngram_size = 3`` table)."""
    tok = np.asarray(tokens).reshape(-1)
    if tok.size == 0:
        return tuple(np.zeros((0, table.heads_per_ngram), dtype=np.int64) for _ in range(table.ngram_size - 1))
    rows = table.rows(torch.as_tensor(tok.astype(np.int64))).cpu().numpy().astype(np.int64)
    k = table.heads_per_ngram
    return tuple(rows[:, o * k:(o + 1) * k] for o in range(table.ngram_size - 1))


def iter_blocks(tokens: np.ndarray, block: int = BLOCK_TOKENS, overlap: int = 2) -> Iterator[tuple[int, np.ndarray]]:
    """``(offset, tokens[offset-overlap : offset+block])`` -- ``overlap``
    tokens of history (none on the first block; ``engraft/damage.py:107-118``
    uses 2, the context of a trigram table)."""
    n = len(tokens)
    offset = 0
    first = True
    while offset < n:
        this_block = min(block, n - offset)
        start = offset if first else offset - overlap
        yield offset, tokens[start:offset + this_block]
        offset += this_block
        first = False


def compute_rows_delta(table, rows_global: np.ndarray, data: np.ndarray) -> dict:
    """``(dnorm, ratio, cos)`` of every overlay row against its true row
    (``engraft/damage.py:126-151``); the true rows come from the device
    gather."""
    true = _read_true_rows(table, np.asarray(rows_global).tolist())
    data = np.asarray(data, dtype=np.float32)
    diff = data.astype(np.float64) - true.astype(np.float64)
    dnorm = np.linalg.norm(diff, axis=1).astype(np.float32)
    norm_true = np.linalg.norm(true, axis=1).astype(np.float64)
    norm_ov = np.linalg.norm(data, axis=1).astype(np.float64)
    ratio = np.where(norm_true > 0, norm_ov / np.maximum(norm_true, 1e-30), np.nan).astype(np.float32)
    denom = norm_ov * norm_true
    dot = np.sum(data.astype(np.float64) * true.astype(np.float64), axis=1)
    cos = np.where(denom > 0, dot / np.maximum(denom, 1e-30), np.nan).astype(np.float32)
    return {"rows_global": np.asarray(rows_global, dtype=np.int32), "dnorm": dnorm, "ratio": ratio, "cos": cos,
            "true": true}


_FILL_POOL = None


def _fill(dst: np.ndarray, src: np.ndarray) -> None:
    """dst[:] = src (converting to dst's type), in 1M-token pieces over four
    threads: numpy's copy releases the GIL, and one thread moves an 8M-token
    block at well under the host's memory bandwidth."""
    global _FILL_POOL
    piece = 1 << 20
    if src.shape[0] <= piece:
        dst[:] = src
        return
    if _FILL_POOL is None:
        from concurrent.futures import ThreadPoolExecutor
        _FILL_POOL = ThreadPoolExecutor(4, thread_name_prefix="eg-fill")
    list(_FILL_POOL.map(lambda i: np.copyto(dst[i:i + piece], src[i:i + piece], casting="unsafe"),
                        range(0, src.shape[0], piece)))


def scan_hits(tokens: np.ndarray, table, overlay_sorted: np.ndarray, dnorm_sorted: np.ndarray,
              block: int = BLOCK_TOKENS) -> dict:
    """Positions of ``tokens`` that read at least one row of the sorted overlay
    ids (``engraft/damage.py:159-224``): ``pos`` / ``n_hit_rows`` /
    ``dnorm_max`` / ``dnorm_sum`` per hit position (the corpus's last
    position excluded), and ``read_count`` per overlay row."""
    tokens = np.asarray(tokens).reshape(-1)
    n = int(tokens.shape[0])
    dev = table.device
    ov = np.asarray(overlay_sorted, dtype=np.int64).reshape(-1)
    n_ov = int(ov.shape[0])
    if n_ov > 1 and np.any(ov[1:] <= ov[:-1]):
        raise ValueError("scan_hits: overlay_sorted must be strictly ascending")
    if n_ov and (ov[0] < 0 or ov[-1] > np.iinfo(np.int32).max):
        raise ValueError("scan_hits: overlay ids must be global rows in [0, 2^31)")
    ids = torch.as_tensor(ov.astype(np.int32), device=dev)
    dn = torch.as_tensor(np.asarray(dnorm_sorted, dtype=np.float32).reshape(-1), device=dev)
    if dn.numel() != n_ov:
        raise ValueError("scan_hits: dnorm_sorted must match overlay_sorted")
    counts = torch.zeros(max(n_ov, 1), dtype=torch.int64, device=dev)
    hist = table.ngram_size - 1
    if block < max(hist, 1):
        # a later block's history would start before the corpus (the
        # reference's loop reads a wrapped-around slice there)
        raise ValueError(f"scan_hits: block ({block}) must be at least the n-gram history ({hist})")
    pos_parts, nh_parts, dmax_parts, dsum_parts = [], [], [], []
    t0 = time.time()
    spec = table.c_spec
    # membership bitmap over the table's rows: almost every lookup is a miss,
    # settled by one bit instead of the binary search
    n_bits = max(int(table.n_rows), 1)
    bitmap = torch.empty(int(_lib.load().eg_id_bitmap_words(n_bits)), dtype=torch.int32, device=dev)
    if n_ov:
        _lib.call("eg_build_id_bitmap", _lib.ptr(ids), n_ov, _lib.ptr(bitmap), n_bits, _lib.stream_ptr(dev))
    # int32 token arrays (a tokenized corpus file) go to the device as they are
    # (4 bytes a token); any other integer type as int64.  Blocks are uploaded
    # on a second stream: block i+1 crosses PCIe while block i is scanned.
    narrow = tokens.dtype == np.int32
    tdt = torch.int32 if narrow else torch.int64
    main = torch.cuda.current_stream(dev)
    upload_stream = torch.cuda.Stream(device=dev)
    blocks = list(iter_blocks(tokens, block=block, overlap=hist))
    # two pinned host buffers (torch's host allocator keeps them for the next
    # call): one is filled while the other's copy to the device is in flight
    cap = max((len(b) for _, b in blocks), default=0)
    staging = [torch.empty(max(cap, 1), dtype=tdt, pin_memory=True) for _ in range(2)] if n_ov else None
    copied = [None, None]  # the last copy out of each pinned buffer

    def upload(j):
        blk = blocks[j][1]
        host = staging[j % 2][:len(blk)]
        if copied[j % 2] is not None:
            copied[j % 2].synchronize()  # that buffer's previous block has left it
        _fill(host.numpy(), blk)
        with torch.cuda.stream(upload_stream):
            t = torch.empty(len(blk), dtype=tdt, device=dev)
            t.copy_(host, non_blocking=True)
            copied[j % 2] = upload_stream.record_event()
        return t, copied[j % 2]

    nxt = upload(0) if blocks and n_ov else None
    for i, (offset, blk) in enumerate(blocks):
        if nxt is None:
            break
        tok, ready = nxt
        main.wait_event(ready)
        tok.record_stream(main)  # allocated on the upload stream, read on this one
        start_local = 0 if offset == 0 else hist
        m = tok.numel() - start_local
        if m > 0:
            # one fused launch: hash, membership, per-position reductions, read
            # counts; n_hit / dnorm_max / dnorm_sum land in the rows of one
            # [3, m] buffer so the hits leave the device in one gather
            out = torch.empty((3, m), dtype=torch.int32, device=dev)
            _lib.call("eg_scan_overlay", ctypes.byref(spec), _lib.ptr(tok), tok.element_size(), tok.numel(),
                      start_local, _lib.ptr(ids), n_ov, _lib.ptr(bitmap), n_bits, _lib.ptr(dn), _lib.ptr(out[0]),
                      _lib.ptr(out[1]), _lib.ptr(out[2]), _lib.ptr(counts), _lib.stream_ptr(dev))
        nxt = upload(i + 1) if i + 1 < len(blocks) else None  # while the scan runs
        lim = min(m, n - 1 - offset)  # the corpus's last position is not a hit
        if lim <= 0:
            continue
        hit_local = torch.nonzero(out[0, :lim] > 0).reshape(-1)
        if hit_local.numel() == 0:
            continue
        vals = out[:, hit_local].cpu().numpy()
        pos_parts.append(hit_local.cpu().numpy() + offset)
        nh_parts.append(vals[0])
        dmax_parts.append(vals[1].view(np.float32))
        dsum_parts.append(vals[2].view(np.float32))
    read_count = counts[:n_ov].cpu().numpy().astype(np.int64)
    dt = time.time() - t0

    def _cat(parts, dtype):
        return np.concatenate(parts) if parts else np.zeros(0, dtype=dtype)

    return {"pos": _cat(pos_parts, np.int64), "n_hit_rows": _cat(nh_parts, np.int32),
            "dnorm_max": _cat(dmax_parts, np.float32), "dnorm_sum": _cat(dsum_parts, np.float32),
            "read_count": read_count, "scan_time_s": dt, "n_tokens": n}
