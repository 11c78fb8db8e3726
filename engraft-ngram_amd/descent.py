"""Descent on the overlay rows: the drop-in for the optimizer core of the
reference (``engraft/replica/distill.py:378-453`` row variables,
``engraft/descend_corpus.py:776-790, 921-947`` the step).

* ``_read_true_rows`` / ``build_rows_var`` -- the variable rows and their start
  values, read from the device table (same names, arguments and errors).
* ``scatter_grad`` -- the gradient of the variables from ``d_out`` and the slot
  row ids: the autograd of ``rows_var[idx_r]`` + ``index_put``
  (``engraft/replica/seq.py:433-441``), computed on the device by grouping
  the slots per variable (counts, range starts, a scatter at start + rank)
  and a reduction of each variable's slots in ascending slot order -- bitwise
  repeatable.
* ``DescentState`` -- ``rows_var`` (fp32 master rows), Adam moments and a
  requantised copy in HBM; ``step`` runs scatter + Adam (torch's single-tensor
  order, fp32) + requantisation in one call (``eg_descent_step``), in the
  reference's dense mode (every variable steps, ``torch.optim.Adam([rows_var])``)
  or the sparse mode of the benchmark's config 2 (only the rows this batch hit).
"""
from __future__ import annotations

import ctypes
import math

import numpy as np
import torch

from . import _lib
from .overlay import DeviceOverlay
from .table import DeviceTable, RowStore

# Locality policies of the variable rows (engraft/replica/distill.py:401-437):
# policy -> (row-set keys whose union is taken, row-set keys removed from it).
_POLICY_RULES: dict[str, tuple[tuple[str, ...], tuple[str, ...]]] = {
    "all-read": (("all_read",), ()),
    "private": (("all_read",), ("neutral_read",)),
    "entity": (("entity", "terme"), ()),
    "t8-answer": (("t8_answer",), ()),
}
_POLICIES = tuple(_POLICY_RULES)


class _Workspace:
    """Grow-only device workspace for the backward kernels, one per (device,
    stream): calls on one stream run in order and may share it; calls on
    different streams get different buffers, so they never race on it.  A
    buffer that is replaced by a larger one was allocated and used on the same
    stream, so torch's allocator reuses its memory only after that stream's
    earlier work."""

    def __init__(self):
        self._buf: dict[tuple[torch.device, int], torch.Tensor] = {}

    def get(self, n_slots: int, n_var: int, device) -> torch.Tensor:
        need = int(_lib.load().eg_backward_workspace_size(int(n_slots), int(n_var)))
        dev = torch.device(device)
        key = (dev, _lib.stream_ptr(dev))
        buf = self._buf.get(key)
        if buf is None or buf.numel() < need:
            buf = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
            self._buf[key] = buf
        return buf


_WS = _Workspace()


def _dout_args(d_out: torch.Tensor):
    if d_out.dtype == torch.bfloat16:
        return 0
    if d_out.dtype == torch.float32:
        return 1
    raise ValueError(f"d_out must be bf16 or f32, got {d_out.dtype}")


def scatter_grad(d_out: torch.Tensor, rows: torch.Tensor, ids: torch.Tensor, dim: int,
                 grad: torch.Tensor | None = None) -> torch.Tensor:
    """Gradient of the variables ``ids`` (sorted unique int32 global rows):
    ``grad[k] = sum over slots (p, h) with rows[p, h] == ids[k] of
    d_out[p, h*dim:(h+1)*dim]`` (f32 ``[len(ids), dim]``; accumulated into
    ``grad`` when given)."""
    dev = d_out.device
    rows = rows.to(device=dev, dtype=torch.int32).contiguous()
    n_pos, heads = rows.shape
    if d_out.numel() != n_pos * heads * dim or not d_out.is_contiguous():
        raise ValueError(f"d_out must be contiguous with {n_pos}x{heads * dim} elements")
    ids = ids.to(device=dev, dtype=torch.int32).contiguous()
    if grad is None:
        grad = torch.zeros((ids.numel(), dim), dtype=torch.float32, device=dev)
    elif grad.shape != (ids.numel(), dim) or grad.dtype != torch.float32 or not grad.is_contiguous():
        raise ValueError("grad must be a contiguous f32 [len(ids), dim] tensor")
    ws = _WS.get(n_pos * heads, ids.numel(), dev)
    _lib.call("eg_scatter_grad", _lib.ptr(d_out), _dout_args(d_out), _lib.ptr(rows), n_pos, heads, dim,
              _lib.ptr(ids), ids.numel(), _lib.ptr(grad), _lib.ptr(ws), ws.numel(), _lib.stream_ptr(dev))
    return grad


class DescentState:
    """Overlay variables and their Adam state, resident in HBM.

    ``ids`` int32 ``[R]`` sorted unique global rows (``row_map`` keys, whose
    values are ``0..R-1`` in ascending id order as ``build_rows_var`` makes
    them); ``master`` f32 ``[R, D]`` (``rows_var``); ``m``/``v`` the moments;
    ``quant`` the requantised copy the forward reads (``None``: keep fp32 only)."""

    def __init__(self, ids: torch.Tensor, master: torch.Tensor, quant_fmt: str | None = "q8_0",
                 base: DeviceTable | None = None, anchor: torch.Tensor | None = None):
        if ids.dtype != torch.int32 or ids.dim() != 1:
            raise ValueError("ids must be a 1-D int32 tensor")
        if master.dtype != torch.float32 or master.dim() != 2 or master.shape[0] != ids.numel():
            raise ValueError("master must be f32 [len(ids), D]")
        if ids.numel() > 1 and not bool((ids[1:] > ids[:-1]).all()):
            raise ValueError("ids must be sorted ascending and unique")
        self.ids = ids.contiguous()
        self.dim = int(master.shape[1])
        dev = master.device
        # master, m and v of a variable side by side: one [R][3][D] buffer whose
        # three [R, D] views the kernels read and write as one run a variable
        # (eg_descent_state.row_stride = 3 D; a config-2 step 3 % faster than
        # three separate arrays)
        self._state = torch.zeros((ids.numel(), 3, self.dim), dtype=torch.float32, device=dev)
        self._state[:, 0] = master
        self.master, self.m, self.v = self._state[:, 0], self._state[:, 1], self._state[:, 2]
        self.stamp = torch.zeros(ids.numel(), dtype=torch.int32, device=dev)
        self.step_count = 0
        self.base = base
        self.quant = RowStore.empty(quant_fmt, ids.numel(), self.dim, dev) if quant_fmt else None
        if self.quant is not None and ids.numel():
            # every variable's quantised row is valid before its first step
            self._requant(master.contiguous(), None)
        # open-addressing index of the ids for the backward's lookups (built
        # once), at most a quarter full: a wavefront's lookups probe in
        # lockstep, so the longest probe chain of 64 lanes sets their time
        cap = 64
        while cap < 4 * ids.numel():
            cap *= 2
        self.index = torch.empty(cap, dtype=torch.int64, device=dev)
        _lib.call("eg_build_row_index", _lib.ptr(self.ids), ids.numel(), _lib.ptr(self.index), cap,
                  _lib.stream_ptr(dev))
        # rows0 of the pull term mu*||rows_var - rows0||^2/||rows0||^2: the anchor
        # rows when given (engraft/descend_corpus.py:780-781, 935-939: rows0 are
        # the starting rows, a warm start's included), else the true rows, read
        # by the step kernel from the base table (engraft/replica/descend.py:141,
        # 252).  The denominator comes from the same rows as the anchor.
        if anchor is not None:
            if anchor.dtype != torch.float32 or tuple(anchor.shape) != tuple(self.master.shape):
                raise ValueError("anchor must be f32 [len(ids), D] like master")
            self.anchor = anchor.to(self.master.device).contiguous()
            rows0 = self.anchor
        else:
            self.anchor = None
            rows0 = base.gather(self.ids.reshape(-1, 1)) if (base is not None and ids.numel()) else self.master
        self.rows0_sq = float(rows0.pow(2).sum().clamp_min(1e-12).item()) if ids.numel() else 0.0

    @property
    def n(self) -> int:
        return int(self.ids.numel())

    @property
    def device(self) -> torch.device:
        return self.master.device

    @classmethod
    def from_rows(cls, table: DeviceTable, rows, quant_fmt: str | None = "q8_0") -> "DescentState":
        """Variables = every distinct row in ``rows`` (e.g. the forward's slot ids),
        started from their true (dequantised) table values."""
        r = rows if isinstance(rows, torch.Tensor) else torch.as_tensor(np.asarray(rows))
        ids = torch.unique(r.to(device=table.device, dtype=torch.int64).reshape(-1)).to(torch.int32)
        master = table.gather(ids.reshape(-1, 1)) if ids.numel() else torch.zeros(
            (0, table.row_len), dtype=torch.float32, device=table.device)
        return cls(ids, master, quant_fmt=quant_fmt, base=table)

    def c_state(self) -> _lib.EgDescentState:
        s = _lib.EgDescentState()
        s.n = self.n
        s.dim = self.dim
        s.ids = _lib.ptr(self.ids)
        s.master = _lib.ptr(self.master)
        s.m = _lib.ptr(self.m)
        s.v = _lib.ptr(self.v)
        s.stamp = _lib.ptr(self.stamp)
        s.row_stride = 3 * self.dim
        if self.quant is not None:
            s.quant = self.quant.c_table()
        s.index = _lib.ptr(self.index)
        s.index_capacity = self.index.numel()
        return s

    def _requant(self, src: torch.Tensor, dst_rows: torch.Tensor | None) -> None:
        tab = self.quant.c_table()
        _lib.call("eg_quantize_rows", _lib.ptr(src), src.shape[0], self.dim,
                  _lib.ptr(dst_rows) if dst_rows is not None else None, ctypes.byref(tab),
                  _lib.stream_ptr(self.device))

    def plan(self, rows: torch.Tensor | None = None, plan: "DescentPlan | None" = None, *,
             slot_var: torch.Tensor | None = None) -> "DescentPlan":
        """The slot grouping of a step over ``rows`` (int32 ``[n_pos, heads]``),
        made now on the current stream (``eg_descent_plan``) for a later
        ``step(..., plan=...)``.  It depends only on the row ids, which the hash
        fixes from the tokens, so a loop can plan the next batch on a second
        stream while the current step runs.  ``plan``: an earlier plan whose
        buffer is reused (its step must have been issued, and ordered before
        this call by the caller when the streams differ).

        ``slot_var`` in place of ``rows``: each slot's variable (a row of
        ``ids``; any other value for none), as ``PreparedForward(...,
        return_slot_vars=True)`` writes them for ``self.overlay()`` -- the
        grouping then needs no row lookup (``eg_descent_plan_slots``)."""
        dev = self.device
        if (rows is None) == (slot_var is None):
            raise ValueError("give rows or slot_var")
        direct = slot_var is not None
        rows = (slot_var if direct else rows).to(device=dev, dtype=torch.int32).contiguous()
        if rows.dim() != 2:
            raise ValueError("rows / slot_var must be [n_pos, heads]")
        n_pos, heads = rows.shape
        need = int(_lib.load().eg_backward_workspace_size(n_pos * heads, self.n))
        ws = plan.workspace if plan is not None and plan.workspace.numel() >= need else \
            torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
        st = self.c_state()
        # the plan's buffers are used on this stream: the caching allocator must not hand
        # them out elsewhere before its work is done, even when the plan is dropped unused
        cur = torch.cuda.current_stream(dev)
        ws.record_stream(cur)
        rows.record_stream(cur)
        _lib.call("eg_descent_plan_slots" if direct else "eg_descent_plan", _lib.ptr(rows), n_pos, heads,
                  ctypes.byref(st), _lib.ptr(ws), ws.numel(), _lib.stream_ptr(dev))
        return DescentPlan(self, rows, ws)

    def step(self, d_out: torch.Tensor, rows: torch.Tensor | None = None, *, lr: float, betas=(0.9, 0.999),
             eps: float = 1e-8, dense: bool = False, mu: float = 0.0, frozen=None, no_alloc: bool = False,
             plan: "DescentPlan | None" = None, slot_var: torch.Tensor | None = None) -> None:
        """One optimizer step from ``d_out`` (bf16/f32 ``[n_pos, heads*D]``) and the
        slots' row ids ``rows`` (int32 ``[n_pos, heads]``).  ``mu``: the pull
        term ``mu*||rows_var - rows0||^2/||rows0||^2`` (rows0 = the state's
        ``anchor`` rows, or the base table's rows of the ids without one).

        ``frozen``: bool ``[R]``, the variables held at their true rows -- the
        masked step of ``engraft/replica/descend.py:262-271`` (``row_mask`` =
        ``~frozen``): their gradient, pull term included, is zero (Adam still
        decays their moments in the dense mode) and their rows are the base
        table's again after the step.

        ``no_alloc``: the step's C call is ``eg_descent_step_noalloc``, which
        allocates nothing (its scratch is a static 16 MiB array per GPU; larger
        steps raise ``EgError``).

        ``plan``: the grouping made by ``plan(rows)`` of this state (``rows``
        may then be omitted); the step is then ``eg_descent_apply`` on it,
        bitwise the same as a step that groups the slots itself.  The caller
        orders the plan's stream before this one.

        ``slot_var`` in place of ``rows``: the slots' variables (see ``plan``);
        the step groups them without a row lookup."""
        dev = self.device
        if slot_var is not None:
            if rows is not None or plan is not None or frozen is not None or no_alloc:
                raise ValueError("slot_var takes neither rows, a plan, frozen rows nor no_alloc")
            plan = self.plan(slot_var=slot_var)
        if plan is not None:
            if plan.state is not self:
                raise ValueError("the plan was made for another DescentState")
            if frozen is not None or no_alloc:
                raise ValueError("a planned step takes neither frozen rows nor no_alloc")
            if rows is not None and (tuple(rows.shape) != tuple(plan.rows.shape)):
                raise ValueError("rows differ in shape from the plan's")
            rows = plan.rows
        if rows is None:
            raise ValueError("rows (or a plan) are required")
        rows = rows.to(device=dev, dtype=torch.int32).contiguous()
        n_pos, heads = rows.shape
        fidx = rows0_f = None
        if frozen is not None:
            fz = torch.as_tensor(np.asarray(frozen.cpu() if isinstance(frozen, torch.Tensor) else frozen, dtype=bool))
            if fz.dim() != 1 or fz.numel() != self.n:
                raise ValueError(f"frozen must be a bool mask over the {self.n} variables")
            if self.base is None:
                raise ValueError("frozen rows are restored from the base table (DescentState(base=...))")
            fidx = fz.nonzero().reshape(-1).to(dev)
            if fidx.numel():
                frozen_ids = self.ids[fidx]
                rows0_f = self.base.gather(frozen_ids.reshape(-1, 1)).reshape(-1, self.dim)
                # at rows0 the pull gradient is exactly zero; slots that read a frozen row carry none
                self.master[fidx] = rows0_f
                rows = torch.where(torch.isin(rows, frozen_ids), torch.full_like(rows, -1), rows)
            else:
                fidx = None
        if d_out.numel() != n_pos * heads * self.dim or not d_out.is_contiguous() or d_out.device != dev:
            raise ValueError(f"d_out must be contiguous on {dev} with {n_pos}x{heads * self.dim} elements")
        opt = _lib.EgAdam()
        opt.lr, opt.beta1, opt.beta2, opt.eps = float(lr), float(betas[0]), float(betas[1]), float(eps)
        opt.step = self.step_count + 1
        opt.dense = 1 if dense else 0
        base = None
        if mu != 0.0:
            if self.anchor is not None:
                opt.anchor = _lib.ptr(self.anchor)
            elif self.base is None:
                raise ValueError("the pull term needs its rows0: DescentState(base=...) or (anchor=...)")
            else:
                base = self.base.c_table
            opt.l2_coef = float(np.float32(mu) / np.float32(self.rows0_sq))
        st = self.c_state()
        if plan is not None:
            ws = plan.workspace
            ws.record_stream(torch.cuda.current_stream(dev))  # freed only after this stream's use
            _lib.call("eg_descent_apply", _lib.ptr(d_out), _dout_args(d_out), n_pos, heads, ctypes.byref(st),
                      ctypes.byref(opt), ctypes.byref(base) if base is not None else None, _lib.ptr(ws), ws.numel(),
                      _lib.stream_ptr(dev))
        elif no_alloc:
            # eg_descent_step_noalloc: the grouping scratch is the library's
            # static per-GPU array (calls overlapping on one GPU race)
            _lib.call("eg_descent_step_noalloc", _lib.ptr(d_out), _dout_args(d_out), _lib.ptr(rows), n_pos, heads,
                      ctypes.byref(st), ctypes.byref(opt), ctypes.byref(base) if base is not None else None,
                      _lib.stream_ptr(dev))
        else:
            ws = _WS.get(n_pos * heads, self.n, dev)
            _lib.call("eg_descent_step", _lib.ptr(d_out), _dout_args(d_out), _lib.ptr(rows), n_pos, heads,
                      ctypes.byref(st), ctypes.byref(opt), ctypes.byref(base) if base is not None else None,
                      _lib.ptr(ws), ws.numel(), _lib.stream_ptr(dev))
        self.step_count += 1  # only once the step is on its way (a rejected call leaves the count)
        if fidx is not None:
            # engraft/replica/descend.py:269-271: the frozen rows are restored after the step
            self.master[fidx] = rows0_f
            if self.quant is not None:
                self._requant(rows0_f.contiguous(), fidx.to(torch.int32))

    def overlay(self, quantized: bool = True) -> DeviceOverlay:
        """The variables as a forward overlay: the requantised rows, or the fp32
        master rows (the reference's ``.pleo`` semantics; a copy of them as they
        are now, since the state keeps master beside its moments)."""
        if quantized and self.quant is not None:
            return DeviceOverlay(self.ids, self.quant, ids_checked=True)
        return DeviceOverlay(self.ids, RowStore("f32", self.dim, self.master.contiguous()), ids_checked=True)


class DescentPlan:
    """The slot grouping of one descent step (``DescentState.plan``): the rows
    it was made from and the device buffer holding it.  A buffer holds one plan;
    ``DescentState.plan(rows, plan=this)`` regroups into it."""

    def __init__(self, state: DescentState, rows: torch.Tensor, workspace: torch.Tensor):
        self.state = state
        self.rows = rows
        self.workspace = workspace


# ---------------------------------------------------------------------------------------------
# Row variables (engraft/replica/distill.py:378-453)
# ---------------------------------------------------------------------------------------------

def true_rows_device(table: DeviceTable, rows_global) -> torch.Tensor:
    """TRUE (dequantised) rows for global ids in any order, as a device f32
    tensor ``[n, row_len]``; ``ValueError`` for an id outside every head
    (``engraft/replica/distill.py:378-395``)."""
    g = np.asarray(list(rows_global) if not isinstance(rows_global, np.ndarray) else rows_global,
                   dtype=np.int64).reshape(-1)
    offsets = np.asarray(table.head_offsets, dtype=np.int64)
    ends = offsets + np.asarray(table.head_vocab_sizes, dtype=np.int64)
    h = np.clip(np.searchsorted(offsets, g, side="right") - 1, 0, len(offsets) - 1)
    bad = ~((offsets[h] <= g) & (g < ends[h]))
    if bad.any():
        raise ValueError(f"_read_true_rows: global row {int(g[bad][0])} outside all heads")
    if g.size == 0:
        return torch.zeros((0, table.row_len), dtype=torch.float32, device=table.device)
    return table.gather(torch.as_tensor(g.astype(np.int32), device=table.device).reshape(-1, 1))


def _read_true_rows(table: DeviceTable, rows_global) -> np.ndarray:
    """``engraft/replica/distill.py:378-395``: the true rows as host f32 ``[n, row_len]``."""
    return true_rows_device(table, rows_global).cpu().numpy()


def build_rows_var(table: DeviceTable, sequences: list[list[int]], policy: str, row_sets: dict,
                   exclude_positions: dict | None = None) -> tuple[dict, torch.Tensor]:
    """``(row_map, rows_var)`` for a locality policy (``engraft/replica/distill.py:
    401-453``): variable rows by policy minus every row read at an excluded
    position; ``row_map`` = ``{global_row: index}`` in ascending row order;
    ``rows_var`` f32 ``[R, row_len]`` (CPU, like the reference) holding the TRUE
    values."""
    rule = _POLICY_RULES.get(policy)
    if rule is None:
        raise ValueError(f"build_rows_var: unknown policy {policy!r} (expected: {_POLICIES})")
    include, subtract = rule

    def ids(keys: tuple[str, ...]) -> np.ndarray:
        return np.unique(np.concatenate([np.asarray(row_sets[k], dtype=np.int64).reshape(-1) for k in keys]
                                        + [np.zeros(0, dtype=np.int64)]))

    # rows read at an excluded position (every head of it), hashed on the device
    excluded = [np.zeros(0, dtype=np.int64)]
    for seq_idx, positions in (exclude_positions or {}).items():
        if len(positions):
            excluded.append(table.rows(sequences[seq_idx]).cpu().numpy()[list(positions)].reshape(-1))
    drop = np.union1d(ids(subtract), np.concatenate(excluded))
    selected = np.setdiff1d(ids(include), drop)  # ascending, unique
    row_map = {int(g): i for i, g in enumerate(selected.tolist())}
    if selected.size == 0:
        return row_map, torch.zeros(0, table.row_len, dtype=torch.float32)
    return row_map, torch.from_numpy(_read_true_rows(table, selected).copy())


def descent_lr(rows0: torch.Tensor, lr_scale: float = 1.0) -> float:
    """``engraft/descend_corpus.py:785-789``: ``lr_scale * 0.01 * mean_row_norm / sqrt(row_len)``."""
    if rows0.shape[0] == 0:
        return 0.0
    mean_row_norm = float(rows0.norm(dim=1).mean().item())
    return lr_scale * 0.01 * mean_row_norm / math.sqrt(rows0.shape[1])
