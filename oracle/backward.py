"""Oracle: sparse gradient scatter + optimizer step + requantisation
(TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py).

* ``scatter_grad``  -- the gradient of the overlay variables: autograd of
  ``rows_var[idx_r]`` + ``index_put`` (``engraft/replica/seq.py:433-441``)
  gives ``grad[r] = sum over (t, h) with row_map[rows[t, h]] == r of
  d_emb[t, h, :]``.  The slots of a variable are taken in ascending slot order
  (``slot = t*n_heads + h``) and summed in fp32 with the association the
  device's slot-ordered reduction fixes (``segment_sum``: sequential up to 32
  slots, pieces of 32 grouped mod 8 beyond); ``scatter_grad_exact`` gives the
  fp64 sum.
* ``adam_step``     -- ``torch.optim.Adam`` (``engraft/descend_corpus.py:
  785-790, 947``) restated in fp32 with torch's single-tensor op order; the
  dense mode updates every variable row like the reference, the sparse mode
  only the rows hit in this step (their moments, lazily).

Pinning (tests/test_oracle_forward_backward.py): ``scatter_grad`` against the
fp64 exact sum (error bound), against a plain per-slot loop for segments of at
most 32 slots, and ``segment_sum`` against an independent reshape formulation
for long segments; ``adam_step``
dense against ``torch.optim.Adam`` itself on CPU (the library routine the
reference calls), multi-step, and the first-step closed form
``p - lr*g/(|g| + eps)`` (m_hat = g, v_hat = g**2).
"""
from __future__ import annotations

import math

import numpy as np


def slot_keys(rows, ids_sorted) -> np.ndarray:
    """Variable index of every slot (``-1`` = frozen row), ``[P*Hh]``."""
    flat = np.asarray(rows, dtype=np.int64).reshape(-1)
    ids = np.asarray(ids_sorted, dtype=np.int64)
    if ids.size == 0:
        return np.full(flat.shape, -1, dtype=np.int64)
    pos = np.searchsorted(ids, flat)
    posc = np.clip(pos, 0, ids.size - 1)
    return np.where(ids[posc] == flat, posc, -1)


PIECE = 32        # slots per piece of a long segment
LONG_GROUPS = 8   # piece sums are accumulated per group j mod 8


def _seq_sum(x: np.ndarray) -> np.ndarray:
    """((0 + x[0]) + x[1]) + ... in fp32, one addition at a time."""
    acc = np.zeros(x.shape[1:], dtype=np.float32)
    for row in x:
        acc = (acc + row).astype(np.float32)
    return acc


def segment_sum(vals: np.ndarray) -> np.ndarray:
    """Sum of one variable's slot gradients ``vals [L, D]`` (ascending slot order)
    with the association the device uses: a segment of at most 32 slots is summed
    in order; a longer one is cut into pieces of 32 slots (each summed in order),
    piece j is added (in order of j) to group ``j mod 8``'s sum, and the eight
    group sums are added in group order."""
    vals = np.asarray(vals, dtype=np.float32)
    n = vals.shape[0]
    if n <= PIECE:
        return _seq_sum(vals)
    pieces = [_seq_sum(vals[j:j + PIECE]) for j in range(0, n, PIECE)]
    groups = []
    for g in range(LONG_GROUPS):
        acc = np.zeros(vals.shape[1:], dtype=np.float32)
        for j in range(g, len(pieces), LONG_GROUPS):
            acc = (acc + pieces[j]).astype(np.float32)
        groups.append(acc)
    tot = groups[0]
    for g in range(1, LONG_GROUPS):
        tot = (tot + groups[g]).astype(np.float32)
    return tot


def scatter_grad(d_emb, rows, ids_sorted) -> tuple[np.ndarray, np.ndarray]:
    """``(grad f32 [R, D], hits int64 [R])``: each variable's slots in ascending
    slot order, summed with ``segment_sum``'s association (sequential for the
    segments of at most 32 slots, which ``np.add.at`` does in index order)."""
    rows = np.asarray(rows, dtype=np.int64)
    return scatter_grad_keys(d_emb, slot_keys(rows, ids_sorted), rows.shape[1],
                             int(np.asarray(ids_sorted).size))


def scatter_grad_keys(d_emb, keys, heads: int, n_var: int) -> tuple[np.ndarray, np.ndarray]:
    """``scatter_grad`` with the variable of every slot given directly
    (``keys [P*heads]``, ``-1`` or ``>= n_var`` = no variable): the gradient of
    ``rows_var`` through ``base.index_put((idx_t, idx_h), rows_var[idx_r])``
    (``engraft/replica/seq.py:433-441``) with ``keys[t*heads + h] = idx_r``."""
    d_emb = np.asarray(d_emb, dtype=np.float32)
    keys = np.asarray(keys, dtype=np.int64).reshape(-1)
    p = keys.size // heads
    d = d_emb.shape[1] // heads if d_emb.size else 0
    grad = np.zeros((n_var, d), dtype=np.float32)
    hits = np.zeros(n_var, dtype=np.int64)
    sel = np.flatnonzero((keys >= 0) & (keys < n_var))
    if sel.size == 0:
        return grad, hits
    order = np.argsort(keys[sel], kind="stable")
    slots = sel[order]
    ks = keys[slots]
    np.add.at(hits, ks, 1)
    flat = d_emb.reshape(p * heads, d)
    short = hits[ks] <= PIECE
    np.add.at(grad, ks[short], flat[slots[short]])  # sequential in index (= slot) order
    for k in np.unique(ks[~short]):
        grad[k] = segment_sum(flat[slots[ks == k]])
    return grad, hits


def scatter_grad_exact(d_emb, rows, ids_sorted) -> np.ndarray:
    d_emb = np.asarray(d_emb, dtype=np.float64)
    rows = np.asarray(rows, dtype=np.int64)
    p, hh = rows.shape
    d = d_emb.shape[1] // hh
    keys = slot_keys(rows, ids_sorted)
    grad = np.zeros((int(np.asarray(ids_sorted).size), d), dtype=np.float64)
    sel = keys >= 0
    np.add.at(grad, keys[sel], d_emb.reshape(p * hh, d)[sel])
    return grad


def adam_step(param, grad, m, v, step: int, lr: float, beta1: float = 0.9, beta2: float = 0.999,
              eps: float = 1e-8, touched=None, rows0=None, l2_coef: float = 0.0):
    """One Adam step (``step`` = the new step count, 1 on the first step).

    fp32, torch single-tensor order: ``m.lerp_(g, 1-b1)``;
    ``v.mul_(b2).addcmul_(g, g, 1-b2)``; ``denom = sqrt(v)/sqrt(1-b2**t) + eps``;
    ``p.addcdiv_(m, denom, -lr/(1-b1**t))``.  ``touched`` (bool ``[R]``) restricts
    the update to those rows (sparse mode); ``None`` updates all rows (dense,
    the reference's ``torch.optim.Adam([rows_var])``).  ``l2_coef`` (fp32
    ``mu / ||rows0||^2``) adds the pull term's gradient
    ``l2_coef * (2 * (p - rows0))`` of ``engraft/descend_corpus.py:935-939`` to
    ``grad`` first (autograd's order: the pow backward ``2 * diff``, then the
    scalar).  Returns new arrays."""
    param = np.array(param, dtype=np.float32, copy=True)
    m = np.array(m, dtype=np.float32, copy=True)
    v = np.array(v, dtype=np.float32, copy=True)
    g = np.asarray(grad, dtype=np.float32)
    sel = slice(None) if touched is None else np.asarray(touched, dtype=bool)
    w1 = np.float32(1.0 - beta1)
    gs, ms, vs, ps = g[sel], m[sel], v[sel], param[sel]
    if l2_coef != 0.0:
        r0 = np.asarray(rows0, dtype=np.float32)[sel]
        gs = (gs + np.float32(l2_coef) * (np.float32(2.0) * (ps - r0))).astype(np.float32)
    ms = (ms + w1 * (gs - ms)).astype(np.float32)
    vs = (vs * np.float32(beta2) + np.float32(1.0 - beta2) * gs * gs).astype(np.float32)
    bc1 = 1.0 - beta1 ** step
    bc2_sqrt = math.sqrt(1.0 - beta2 ** step)
    step_size = np.float32(lr / bc1)
    denom = (np.sqrt(vs) / np.float32(bc2_sqrt) + np.float32(eps)).astype(np.float32)
    ps = (ps + (-step_size) * (ms / denom)).astype(np.float32)
    m[sel], v[sel], param[sel] = ms, vs, ps
    return param, m, v
