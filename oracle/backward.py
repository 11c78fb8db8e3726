"""Oracle: sparse gradient scatter + optimizer step + requantisation
(TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py).

* ``scatter_grad``  -- the gradient of the overlay variables: autograd of
  ``rows_var[idx_r]`` + ``index_put`` (``engraft/replica/seq.py:433-441``)
  gives ``grad[r] = sum over (t, h) with row_map[rows[t, h]] == r of
  d_emb[t, h, :]``.  The sum is taken in ascending slot order
  (``slot = t*n_heads + h``) in fp32, one addition at a time (``np.add.at`` is
  sequential in index order), which is the order the device's sort +
  segmented reduce fixes; ``scatter_grad_exact`` gives the fp64 sum.
* ``adam_step``     -- ``torch.optim.Adam`` (``engraft/descend_corpus.py:
  785-790, 947``) restated in fp32 with torch's single-tensor op order; the
  dense mode updates every variable row like the reference, the sparse mode
  only the rows hit in this step (their moments, lazily).

Pinning (tests/test_oracle_backward.py): ``scatter_grad`` against the fp64
exact sum (error bound) and its permutation invariance as a set; ``adam_step``
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


def scatter_grad(d_emb, rows, ids_sorted) -> tuple[np.ndarray, np.ndarray]:
    """``(grad f32 [R, D], hits int64 [R])`` -- sequential fp32 in slot order."""
    d_emb = np.asarray(d_emb, dtype=np.float32)
    rows = np.asarray(rows, dtype=np.int64)
    p, hh = rows.shape
    d = d_emb.shape[1] // hh
    keys = slot_keys(rows, ids_sorted)
    r = int(np.asarray(ids_sorted).size)
    grad = np.zeros((r, d), dtype=np.float32)
    hits = np.zeros(r, dtype=np.int64)
    sel = keys >= 0
    if sel.any():
        vals = d_emb.reshape(p * hh, d)[sel]
        np.add.at(grad, keys[sel], vals)
        np.add.at(hits, keys[sel], 1)
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
