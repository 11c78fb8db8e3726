"""The differentiable sequence overlay and the per-position true embedding, on
the device: the drop-ins for ``OverlayEmb`` / ``overlay_key_len``
(``engraft/replica/seq.py:222-444``) and ``Replica.ple_true_emb``
(``engraft/replica/model.py:473-495``), and the sequence seam around the
model: ``PatchStats``, ``ple_emb_patched``, ``seq_forward``, ``seq_step``
(``engraft/replica/seq.py:453-637, 809-921, 1340-1470``).

``OverlayEmb.build`` does in a few launches what the reference does with a
per-position Python loop:

1. hash every position (``eg_hash_rows``; with ``segment_ids`` each position
   looks back only to its segment's first token, which is what hashing the
   isolated ``tokens[s(t):]`` gives);
2. resolve every slot's variable (``eg_lookup_rows`` over the sorted int keys
   of ``row_map``), then overwrite the slots of the long ``(window, head)``
   keys, which win over the global row -- host dict lookups, one per
   position, only when ``row_map`` has tuple keys;
3. gather: every slot reads ``rows_var[slot_var]`` or, without a variable, its
   dequantised table row (``eg_gather_slots``), through a C++ autograd
   function (``csrc/eg_autograd.cpp``) whose backward takes no GIL.

The slot plan (rows + slot variables, the part that does not depend on
``rows_var``) is cached per ``(tokens, start, n_positions, segment starts)``
on the instance, and per fragment in the caller's ``overlay_cache`` (FIFO,
4096 entries), like the reference's base cache.  The backward of the gather
sums every variable's slot gradients in ascending slot order,
deterministically (the same association as the descent step's scatter), from
the slots' grouping by variable that the first build wanting a gradient makes
and keeps with the plan (``eg_scatter_grad_plan_slots``, then
``eg_scatter_grad_apply`` every backward).
"""
from __future__ import annotations

import contextlib
import ctypes
import dataclasses
import time

import numpy as np
import torch

from . import _lib
from .overlay import DeviceOverlay
from .pack import seg_starts_from_segment_ids

OVERLAY_CACHE_MAX_ENTRIES = 4096  # engraft/replica/seq.py:182


def overlay_key_len(row_map: dict) -> int | None:
    """Length ``K`` of the long-key windows of ``row_map`` (``None`` without
    tuple keys); all windows must share one length
    (``engraft/replica/seq.py:222-234``, same ``AssertionError``)."""
    lengths = {len(key[0]) for key in row_map if isinstance(key, tuple)}
    if not lengths:
        return None
    assert len(lengths) == 1, f"overlay_key_len: long keys of different lengths in row_map: {lengths}"
    return next(iter(lengths))


def _slot_grouping(plan: dict, n_var: int, dev) -> torch.Tensor:
    """The slots of ``plan`` grouped by variable (``eg_scatter_grad_plan_slots``),
    made once per plan and variable count and kept with the plan: every
    backward of the plan then only sums (``eg_scatter_grad_apply``)."""
    cache = plan.setdefault("grouping", {})
    ws = cache.get(n_var)
    if ws is None:
        slot_var = plan["slot_var"]
        n, heads = slot_var.shape
        need = int(_lib.load().eg_backward_workspace_size(n * heads, n_var))
        ws = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
        _lib.call("eg_scatter_grad_plan_slots", _lib.ptr(slot_var), n, heads, n_var, _lib.ptr(ws), ws.numel(),
                  _lib.stream_ptr(dev))
        cache[n_var] = ws
    return ws


_NO_WS: dict = {}


def _no_grouping(dev) -> torch.Tensor:
    """The empty workspace that stands for "no grouping" on ``dev``."""
    ws = _NO_WS.get(dev)
    if ws is None:
        ws = _NO_WS[dev] = torch.empty(0, dtype=torch.uint8, device=dev)
    return ws


@dataclasses.dataclass
class OverlayEmb:
    """For positions ``start..n_positions-1`` of ``tokens``, the PLE embedding
    ``[n_positions-start, n_heads*row_len]`` with ``row_map``'s rows replaced
    by ``rows_var`` -- differentiable in ``rows_var``, the plain gather
    everywhere else (``engraft/replica/seq.py:237-444``).

    ``row_map`` keys: ``int`` = global row, or ``((K tokens), head)`` = a long
    key that wins over the global row at a position whose last ``K`` tokens
    (all inside its segment) are the window.  Values: rows of ``rows_var``.
    ``n_key_hits`` / ``n_id_hits`` count the slots each kind replaced in the
    last ``build``."""

    table: object
    tokens: list[int]
    rows_var: torch.Tensor
    row_map: dict
    segment_ids: torch.Tensor | None = None
    overlay_cache: dict | None = None

    def __post_init__(self) -> None:
        if isinstance(self.tokens, torch.Tensor):
            self._tok = [int(x) for x in self.tokens.reshape(-1).tolist()]
        else:
            self._tok = [int(x) for x in self.tokens]
        self._plans: dict[tuple, dict] = {}
        self._seg_starts: np.ndarray | None = None
        self._seg_ranges: list[tuple[int, int]] | None = None
        if self.segment_ids is not None:
            starts = seg_starts_from_segment_ids(self.segment_ids)
            self._seg_starts = starts
            bounds = np.flatnonzero(np.diff(starts) != 0) + 1
            edges = [0] + bounds.tolist() + [len(starts)]
            self._seg_ranges = [(edges[i], edges[i + 1]) for i in range(len(edges) - 1) if edges[i + 1] > edges[i]]
        dev = self.table.device
        self._dev = dev
        self._row_len = self.table.row_len
        int_keys = [k for k in self.row_map if not isinstance(k, tuple)]
        ids = np.array(int_keys, dtype=np.int64)
        var = np.array([self.row_map[k] for k in int_keys], dtype=np.int64)
        order = np.argsort(ids, kind="stable")
        ids, var = ids[order], var[order]
        if ids.size and (ids[0] < 0 or ids[-1] > np.iinfo(np.int32).max):
            raise ValueError("row_map int keys must be global rows in [0, 2^31)")
        self._ids = torch.from_numpy(ids.astype(np.int32)).to(dev)
        self._ids_var = torch.from_numpy(var.astype(np.int32)).to(dev)
        self._key_len = overlay_key_len(self.row_map)
        self._windows: dict[tuple, list[tuple[int, int]]] = {}
        for k, r in self.row_map.items():
            if isinstance(k, tuple):
                self._windows.setdefault(tuple(int(x) for x in k[0]), []).append((int(k[1]), int(r)))
        vals = [int(r) for r in self.row_map.values()]
        self._max_var = max(vals) if vals else -1
        if vals and min(vals) < 0:
            raise IndexError("row_map values must be rows of rows_var (>= 0)")
        self.n_key_hits = 0
        self.n_id_hits = 0

    # ---- the slot plan -----------------------------------------------------------------------
    def _plan_tokens(self, tokens: list[int], seg_start: np.ndarray | None, start: int, end: int) -> dict:
        """Rows and slot variables of positions ``start..end-1`` of ``tokens``
        (``seg_start``: per-position segment start, or ``None`` = one sequence)."""
        table = self.table
        dev = table.device
        heads = table.n_heads
        n = end - start
        if n <= 0:
            z = torch.zeros((0, heads), dtype=torch.int32, device=dev)
            return {"rows": z, "slot_var": z.clone(), "n_key_hits": 0, "n_id_hits": 0}
        rows = table.rows(tokens[:end], seg_start=None if seg_start is None else seg_start[:end])[start:].contiguous()
        slot_var = torch.empty_like(rows)
        _lib.call("eg_lookup_rows", _lib.ptr(rows), rows.numel(), _lib.ptr(self._ids), _lib.ptr(self._ids_var),
                  self._ids.numel(), _lib.ptr(slot_var), None, _lib.stream_ptr(dev))
        n_key = 0
        n_overridden_id = 0
        if self._key_len is not None:
            K = self._key_len
            kt: list[int] = []
            kh: list[int] = []
            kr: list[int] = []
            for t in range(max(start, K - 1), end):
                t_local = t - (int(seg_start[t]) if seg_start is not None else 0)
                if t_local < K - 1:
                    continue
                hits = self._windows.get(tuple(tokens[t - K + 1:t + 1]))
                if hits is None:
                    continue
                for h, r in hits:
                    if 0 <= h < heads:
                        kt.append(t - start)
                        kh.append(h)
                        kr.append(r)
            if kt:
                ti = torch.tensor(kt, dtype=torch.int64, device=dev)
                hi = torch.tensor(kh, dtype=torch.int64, device=dev)
                n_overridden_id = int((slot_var[ti, hi] >= 0).sum().item())
                slot_var.index_put_((ti, hi), torch.tensor(kr, dtype=torch.int32, device=dev))
                n_key = len(kt)
        n_id_total = int((slot_var >= 0).sum().item()) if self._ids.numel() or n_key else 0
        return {"rows": rows, "slot_var": slot_var, "n_key_hits": n_key, "n_id_hits": n_id_total - n_key}

    def _plan_fragments(self, n_positions: int) -> dict:
        """The plan assembled fragment by fragment through ``overlay_cache``
        (``engraft/replica/seq.py:324-370``): a fragment's plan depends only on
        its own tokens (its hash never looks before its first token)."""
        rows_parts: list[torch.Tensor] = []
        slot_parts: list[torch.Tensor] = []
        n_key = n_id = 0
        for s_i, e_i in self._seg_ranges or []:
            if s_i >= n_positions:
                break
            frag = tuple(self._tok[s_i:e_i])
            entry = self.overlay_cache.get(frag)
            if entry is None:
                entry = self._plan_tokens(list(frag), None, 0, len(frag))
                sv = entry["slot_var"]
                entry["key_per_pos"] = None
                entry["id_per_pos"] = (sv >= 0).sum(dim=1).cpu().numpy()
                if self._key_len is not None:
                    entry["key_per_pos"] = self._key_hits_per_pos(list(frag))
                if len(self.overlay_cache) >= OVERLAY_CACHE_MAX_ENTRIES:
                    self.overlay_cache.pop(next(iter(self.overlay_cache)))  # FIFO: oldest first
                self.overlay_cache[frag] = entry
            m = min(e_i, n_positions) - s_i
            rows_parts.append(entry["rows"][:m])
            slot_parts.append(entry["slot_var"][:m])
            kpp = entry["key_per_pos"]
            k = int(kpp[:m].sum()) if kpp is not None else 0
            n_key += k
            n_id += int(entry["id_per_pos"][:m].sum()) - k
        heads = self.table.n_heads
        dev = self.table.device
        if rows_parts:
            rows = torch.cat(rows_parts).contiguous()
            slot_var = torch.cat(slot_parts).contiguous()
        else:
            rows = torch.zeros((0, heads), dtype=torch.int32, device=dev)
            slot_var = rows.clone()
        return {"rows": rows, "slot_var": slot_var, "n_key_hits": n_key, "n_id_hits": n_id}

    def _key_hits_per_pos(self, frag: list[int]) -> np.ndarray:
        K = self._key_len
        out = np.zeros(len(frag), dtype=np.int64)
        for t in range(K - 1, len(frag)):
            hits = self._windows.get(tuple(frag[t - K + 1:t + 1]))
            if hits:
                out[t] = sum(1 for h, _ in hits if 0 <= h < self.table.n_heads)
        return out

    # ---- the reference's method ----------------------------------------------------------------
    def build(self, n_positions: int, start: int = 0) -> torch.Tensor:
        if not 0 <= start <= n_positions <= len(self._tok):
            raise IndexError(f"positions [{start}, {n_positions}) outside the {len(self._tok)} tokens")
        rv = self.rows_var
        shape = rv.shape
        row_len, dev = self._row_len, self._dev
        if len(shape) != 2 or shape[1] != row_len:
            raise ValueError(f"rows_var must be [R, {row_len}], got {tuple(shape)}")
        n_var = shape[0]
        if self._max_var >= n_var:
            raise IndexError(f"row_map names row {self._max_var} of a {n_var}-row rows_var")
        if self.overlay_cache is not None and self._seg_ranges is not None and start == 0:
            plan = self._plan_fragments(n_positions)
        else:
            # the tokens and segments are fixed per instance: the range names the plan
            key = (start, n_positions)
            plan = self._plans.get(key)
            if plan is None:
                plan = self._plan_tokens(self._tok, self._seg_starts, start, n_positions)
                self._plans[key] = plan
        self.n_key_hits = plan["n_key_hits"]
        self.n_id_hits = plan["n_id_hits"]
        # out f32 [n, heads * dim] = per slot rows_var[slot_var] or the table row
        # (eg_gather_slots), differentiable in rows_var: its backward sums the
        # output gradient into the variables from the plan's slot grouping
        # (eg_scatter_grad_apply; written whole, a variable no slot reads gets
        # zeros).  A C++ autograd function (csrc/eg_autograd.cpp).
        rows = plan["rows"]
        n = rows.shape[0]
        ws = (_slot_grouping(plan, n_var, dev) if n > 0 and n_var > 0 and rv.requires_grad and torch.is_grad_enabled()
              else _no_grouping(dev))
        ct = self.table.c_table
        out = _lib.autograd_ext().gather_slots(rv, rows, plan["slot_var"], ws, ctypes.addressof(ct), row_len,
                                               _lib.stream_ptr(dev))
        if rv.dtype is not torch.float32 or rv.device != dev:
            out = out.to(device=rv.device, dtype=rv.dtype)
        # [n_positions - start, n_heads * row_len] as the plan's rows are
        return out if out.shape[0] == n_positions - start else out.reshape(n_positions - start, -1)


def _as_overlay(table, overlay) -> DeviceOverlay | None:
    if overlay is None:
        return None
    if isinstance(overlay, DeviceOverlay):
        return overlay
    if not overlay:
        return None
    return DeviceOverlay.from_dict(overlay, table.row_len, device=table.device)


def ple_true_emb(table, tokens: list[int], t: int, overlay=None) -> torch.Tensor:
    """``emb [1, n_heads*row_len]`` f32 of position ``t`` of ``tokens``, the
    rows whose global id is in ``overlay`` (``{global_row: vector}`` or a
    ``DeviceOverlay``) replaced (``engraft/replica/model.py:473-495``).  On
    the table's device."""
    if not 0 <= t < len(tokens):
        raise IndexError(f"position {t} outside [0, {len(tokens)})")
    lo = max(0, t - table.ngram_size + 1)
    return ple_true_emb_range(table, list(tokens[lo:t + 1]), t - lo, t - lo + 1, overlay)


def ple_true_emb_range(table, tokens, start: int, end: int, overlay=None, seg_start=None) -> torch.Tensor:
    """``ple_true_emb`` of positions ``start..end-1`` in one launch: the
    ``torch.cat`` of the per-position loop at ``engraft/replica/model.py:
    845-853``; f32 ``[end-start, n_heads*row_len]``."""
    tok = tokens if isinstance(tokens, torch.Tensor) else torch.as_tensor(np.asarray(tokens, dtype=np.int64))
    rows = table.rows(tok[:end], seg_start=None if seg_start is None else np.asarray(seg_start)[:end])
    return table.gather(rows[start:end].contiguous(), overlay=_as_overlay(table, overlay))


def exclusive_rows_at_position(table, tokens: list[int], n_positions: int, p: int,
                               heads: range | None = None) -> set[int]:
    """Global rows of position ``p`` (among ``heads``, default all) that no
    other position ``0..n_positions-1`` reads (``engraft/replica/seq.py:
    924-941``): the rows over which a sequence gradient can be compared with
    an isolated single-step one.

    One ``eg_hash_rows`` over the whole ``tokens`` stream gives every
    position's rows (position ``t``'s rows depend only on its own n-gram
    window, so this is the reference's per-position ``RowSet`` loop), then a
    set difference on the host.  ``p`` indexes like the reference's list
    index (a negative ``p`` counts from the end and is never skipped as
    "itself"); positions past the stream raise ``IndexError`` as there."""
    heads = heads if heads is not None else range(table.n_heads)
    n_tok = len(tokens)
    if n_tok == 0 or n_positions > n_tok:
        raise IndexError(f"positions [0, {max(n_positions, 1)}) outside a stream of {n_tok} tokens")
    tok = tokens if isinstance(tokens, torch.Tensor) else torch.as_tensor(np.asarray(tokens, dtype=np.int64))
    rows = table.rows(tok).cpu().numpy()
    row_p = rows[p]
    candidates = {int(row_p[h]) for h in heads}
    n = max(int(n_positions), 0)
    others = rows[:n]
    if 0 <= p < n:
        others = np.delete(others, p, axis=0)
    return candidates - set(np.unique(others).tolist())


class ReplicaTableMixin:
    """``Replica.ple_true_emb`` as a method (``engraft/replica/model.py:473-495``):
    a model class that keeps its table in ``self.table``, as the reference's
    ``Replica`` does, inherits it and reads its PLE rows from the device
    table (the rows come back on the table's device, not the CPU)."""

    table = None

    def ple_true_emb(self, tokens: list[int], t: int, overlay=None) -> torch.Tensor:
        return ple_true_emb(self.table, tokens, t, overlay)


# ---------------------------------------------------------------------------------------------
# The sequence seam: the model reads its PLE rows through replica.ple_true_emb
# (engraft/replica/model.py:845-853); a sequence forward shadows that method with
# slices of one precomputed OverlayEmb (engraft/replica/seq.py:570-637, 809-921,
# 1340-1470).  Only the table path's half is here: the model's own patches (MoE
# experts, routing, attention masking of packed segments) belong to the model.
# ---------------------------------------------------------------------------------------------
@dataclasses.dataclass
class PatchStats:
    """Counters proving the ``ple_true_emb`` patch took
    (``engraft/replica/seq.py:453-500``): ``n_ple_calls`` must equal the
    number of new positions ``n_prefix - start``; ``n_key_hits`` /
    ``n_id_hits`` echo the very ``OverlayEmb`` that produced the forward."""

    n_ple_calls: int = 0
    n_key_hits: int = 0
    n_id_hits: int = 0


@contextlib.contextmanager
def ple_emb_patched(replica, precomputed_emb: torch.Tensor, stats: PatchStats, start: int = 0):
    """For the duration of the ``with`` block, ``replica.ple_true_emb`` (an
    instance attribute, shadowing the class method) returns
    ``precomputed_emb[t - start]`` as ``[1, n_embd]`` and counts the call;
    the instance's own attribute (or its absence) is restored in ``finally``
    (the ``ple_true_emb`` part of ``expert_op_patched``,
    ``engraft/replica/seq.py:570-637``)."""
    had = "ple_true_emb" in replica.__dict__
    orig = replica.__dict__.get("ple_true_emb")

    def patched_ple_true_emb(tokens_arg, t, overlay=None):
        stats.n_ple_calls += 1
        return precomputed_emb[t - start].unsqueeze(0)

    replica.ple_true_emb = patched_ple_true_emb
    try:
        yield
    finally:
        if had:
            replica.__dict__["ple_true_emb"] = orig
        else:
            del replica.__dict__["ple_true_emb"]


def _new_positions_start(base_state, cache, tokens) -> tuple[int, object]:
    """``start`` of the new positions (``engraft/replica/seq.py:893-906``): a
    cache hit's or the given ``base_state``'s ``n_prefix``, else 0."""
    n_prefix = len(tokens) - 1
    if cache is not None:
        hit = cache.lookup(list(tokens[:n_prefix]), {})
        if hit is not None:
            return int(hit[0].n_prefix), hit[0]
    if base_state is not None:
        return int(base_state.n_prefix), base_state
    return 0, None


def seq_forward(replica, tokens, rows_var: torch.Tensor, row_map: dict, return_logits: bool = True, *,
                grad_proxy: bool = True, base_state=None, cache=None, segment_ids=None, overlay_cache=None,
                **prefix_kwargs):
    """Sequence forward (``engraft/replica/seq.py:809-921``): ``OverlayEmb``
    over the new positions ``start..n_prefix-1`` (on the device,
    differentiable in ``rows_var``), then ``replica.prefix(tokens, ...)`` with
    ``replica.ple_true_emb`` reading slices of it.  ``ValueError`` with fewer
    than 2 tokens.  Returns ``(state, stats)``; ``stats.n_ple_calls`` is
    ``n_prefix - start`` when the model read every new position through the
    patch.  Further keyword arguments go to ``replica.prefix``."""
    n_prefix = len(tokens) - 1
    if n_prefix <= 0:
        raise ValueError("seq_forward: need at least 2 tokens")
    start, _ = _new_positions_start(base_state, cache, tokens)
    overlay_emb = OverlayEmb(replica.table, tokens, rows_var, row_map, segment_ids=segment_ids,
                             overlay_cache=overlay_cache)
    precomputed = overlay_emb.build(n_prefix, start=start)
    stats = PatchStats(n_key_hits=overlay_emb.n_key_hits, n_id_hits=overlay_emb.n_id_hits)
    with ple_emb_patched(replica, precomputed, stats, start=start):
        state = replica.prefix(tokens, grad_proxy=grad_proxy, return_logits=return_logits, base_state=base_state,
                               cache=cache, **prefix_kwargs)
    return state, stats


def seq_step(replica, tokens, rows_var: torch.Tensor, row_map: dict, loss_fn, *, base_state=None, cache=None,
             segment_ids=None, overlay_cache=None, **prefix_kwargs):
    """Sequence forward + backward with the patch active through
    ``loss.backward()`` (``engraft/replica/seq.py:1340-1470``): the gradient
    reaches ``rows_var`` through the device scatter of ``OverlayEmb``.
    Returns ``(loss, timings, stats)``; ``AssertionError`` when
    ``stats.n_ple_calls != n_prefix - start`` (the patch did not take)."""
    t_entry = time.perf_counter()
    n_prefix = len(tokens) - 1
    if n_prefix <= 0:
        raise ValueError("seq_step_triton: need at least 2 tokens")
    start, _ = _new_positions_start(base_state, cache, tokens)
    overlay_emb = OverlayEmb(replica.table, tokens, rows_var, row_map, segment_ids=segment_ids,
                             overlay_cache=overlay_cache)
    precomputed = overlay_emb.build(n_prefix, start=start)
    stats = PatchStats(n_key_hits=overlay_emb.n_key_hits, n_id_hits=overlay_emb.n_id_hits)
    dev = rows_var.device
    sync = (lambda: torch.cuda.synchronize(dev)) if dev.type == "cuda" else (lambda: None)
    with ple_emb_patched(replica, precomputed, stats, start=start):
        sync()
        t0 = time.perf_counter()
        state = replica.prefix(tokens, grad_proxy=True, return_logits=True, base_state=base_state, cache=cache,
                               **prefix_kwargs)
        sync()
        t_fwd = time.perf_counter() - t0
        loss = loss_fn(state)
        t1 = time.perf_counter()
        loss.backward()
        sync()
        t_bwd = time.perf_counter() - t1
    assert stats.n_ple_calls == n_prefix - start, (
        f"seq_step_triton: n_ple_calls={stats.n_ple_calls} != n_prefix-start={n_prefix - start} "
        "(the ple_true_emb patch did not take -- see PatchStats)")
    return loss, {"fwd_s": t_fwd, "bwd_s": t_bwd, "pre_s": t0 - t_entry}, stats
