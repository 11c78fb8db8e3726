"""Oracle: the PLE block that consumes the gathered rows (TEST
INFRASTRUCTURE ONLY -- see oracle/__init__.py).

* ``ple_forward``  -- torch fp32 on the CPU, step for step as
  ``engraft/replica/layers.py:565-626`` with ``rmsnorm`` (``:22-35``),
  ``rmsnorm_grouped`` (``:37-42``) and the per-position loop of
  ``causal_depthwise_conv`` (``:257-293``).
* ``Replica`` / ``ple_out_numpy`` -- the independent numpy formulation of the
  same block (``PleReplica`` in ``engraft/lens.py:221-415``: fp64 mean of
  squares, the shifted-array convolution with a fixed dilation, the one-token
  continuations of ``ple_out_at`` and the finite-difference Jacobian).

Pinning (tests/test_oracle_ple.py): the two agree within 1e-4 on the real
dimensions (hc 4, n_embd 2560, 4 taps, dilation 3), per position with the
returned history as on the whole sequence, as the reference's own
``tests/test_replica_layers.py:238-282`` checks them; ``Replica`` also passes
the reference's known answers for ``PleReplica`` (``tests/test_lens.py:
210-320``: gate 1/2 at a zero embedding, scale invariance of the gate, a
one-position convolution through the last tap alone, ``ple_out = gated +
conv_out``, ``ple_out_at`` = ``ple_out`` at the true embedding, the Jacobian
against finite differences and, with the convolution zeroed and zero hidden
state, against the closed form ``0.5 * w_value``).
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.to(torch.float32)
    ms = xf.pow(2).mean(dim=-1, keepdim=True)
    return (xf * torch.rsqrt(ms + eps) * weight.to(torch.float32)).to(x.dtype)


def rmsnorm_grouped(x, weight_flat, eps, hc):
    return rmsnorm(x, weight_flat.reshape(hc, x.shape[-1]), eps)


def causal_depthwise_conv(x_new, history, weight, dilation=1):
    kern = weight.shape[1]
    t_len, c = x_new.shape
    full = torch.cat([history, x_new], dim=0)
    hist_len = history.shape[0]
    acc = torch.zeros(t_len, c, dtype=x_new.dtype)
    for k in range(kern):
        back = (kern - 1 - k) * dilation
        w_k = weight[:, k]
        for t in range(t_len):
            src_idx = hist_len + t - back
            if src_idx < 0:
                continue
            acc[t] += full[src_idx] * w_k
    return acc


def ple_forward(emb, hidden, w: dict, hist, hc: int, n_embd: int, eps: float, ngram_size: int,
                detach_value: bool = False, detach_gate: bool = False):
    """Returns ``(out [T, hc, n], new_hist, s [T, hc], gate [T, hc])``;
    ``detach_value`` / ``detach_gate`` detach that factor before ``gated =
    value * gate`` (``layers.py:600-604``)."""
    t_len = emb.shape[0]
    key = (emb @ w["w_key"].T).reshape(t_len, hc, n_embd)
    key = rmsnorm_grouped(key, w["norm_key"], eps, hc)
    query = rmsnorm_grouped(hidden, w["norm_query"], eps, hc)
    s = (key * query).sum(dim=-1) / (n_embd ** 0.5)
    mag = torch.sqrt(torch.clamp(s.abs(), min=1e-6))
    gate = torch.sigmoid(torch.sign(s) * mag)
    value = emb @ w["w_value"].T
    g = gate.detach() if detach_gate else gate
    v = value.detach() if detach_value else value
    gated = v.unsqueeze(1) * g.unsqueeze(-1)
    normed = rmsnorm_grouped(gated, w["norm_conv"], eps, hc)
    normed_flat = normed.reshape(t_len, hc * n_embd)
    hist_flat = hist.reshape(hist.shape[0], hc * n_embd) if hist.numel() else hist.reshape(0, hc * n_embd)
    conv_out = causal_depthwise_conv(normed_flat, hist_flat, w["conv1d"], dilation=ngram_size)
    conv_out = F.silu(conv_out).reshape(t_len, hc, n_embd)
    out = hidden + gated + conv_out
    hist_len = (w["conv1d"].shape[1] - 1) * ngram_size
    hist_full = torch.cat([hist.reshape(-1, hc, n_embd), normed], dim=0)
    new_hist = hist_full[-hist_len:] if hist_len > 0 else hist_full[:0]
    return out, new_hist, s, gate


class Replica:
    """The numpy formulation of the block, method for method as ``PleReplica``
    (``engraft/lens.py:221-415``) with the weights given directly: RMS norms
    with an fp64 mean of squares (``:282-287``), the gate's sign-root and
    sigmoid in fp64 (``:301-312``), the shifted-array convolution over zero
    history (``:318-332``), ``ple_out_at``'s one-token continuations with the
    history taken from the true sequence (``:341-385``) and the
    central-difference Jacobian in blocks of 512 variants (``:387-415``)."""

    def __init__(self, w: dict, hc: int, n_embd: int, eps: float, dilation: int = 3):
        a = lambda x: np.asarray(x, dtype=np.float32)
        self.hc, self.n, self.eps, self.dil = hc, n_embd, float(eps), dilation
        self.w_key = a(w["w_key"])
        self.w_value = a(w["w_value"])
        self.norm_key = a(w["norm_key"]).reshape(hc, n_embd)
        self.norm_query = a(w["norm_query"]).reshape(hc, n_embd)
        self.norm_conv = a(w["norm_conv"]).reshape(hc, n_embd)
        self.taps = a(w["conv1d"]).reshape(hc * n_embd, -1).shape[1]
        self.conv1d = a(w["conv1d"]).reshape(hc, n_embd, self.taps).copy()

    def rms(self, x, weight):
        ms = np.mean(np.asarray(x).astype(np.float64) ** 2, axis=-1, keepdims=True)
        return (x / np.sqrt(ms + self.eps)).astype(np.float32) * weight

    def key(self, emb):
        raw = (np.asarray(emb, dtype=np.float32) @ self.w_key.T).reshape(-1, self.hc, self.n)
        return self.rms(raw, self.norm_key)

    def value(self, emb):
        return (np.asarray(emb, dtype=np.float32) @ self.w_value.T).astype(np.float32)

    def gate(self, emb, hidden):
        k = self.key(emb)
        q = self.rms(np.asarray(hidden, dtype=np.float32), self.norm_query)
        s = (np.sum(k * q, axis=-1) / np.sqrt(self.n)).astype(np.float64)
        root = np.sign(s) * np.sqrt(np.clip(np.abs(s), 1e-6, None))
        return (1.0 / (1.0 + np.exp(-root))).astype(np.float32)

    def gated(self, emb, hidden):
        return (self.value(emb)[:, None, :] * self.gate(emb, hidden)[:, :, None]).astype(np.float32)

    def _silu(self, acc):
        return (acc / (1.0 + np.exp(-acc))).astype(np.float32)

    def conv_out(self, gated_seq):
        normed = self.rms(np.asarray(gated_seq, dtype=np.float32), self.norm_conv)
        t_len = normed.shape[0]
        acc = np.zeros_like(normed)
        for k in range(self.taps):
            back = (self.taps - 1 - k) * self.dil
            w_k = self.conv1d[:, :, k]
            if back == 0:
                acc += normed * w_k[None]
            elif back < t_len:
                sh = np.zeros_like(normed)
                sh[back:] = normed[:t_len - back]
                acc += sh * w_k[None]
        return self._silu(acc)

    def ple_out(self, emb_seq, hidden_seq):
        g = self.gated(emb_seq, hidden_seq)
        return (g + self.conv_out(g)).astype(np.float32)

    def ple_out_at(self, emb_t, emb_seq, hidden_seq, t: int):
        emb_t = np.asarray(emb_t, dtype=np.float32)
        b = emb_t.shape[0]
        hid = np.broadcast_to(np.asarray(hidden_seq, dtype=np.float32)[t], (b, self.hc, self.n))
        g_b = (self.value(emb_t)[:, None, :] * self.gate(emb_t, hid)[:, :, None]).astype(np.float32)
        normed_true = self.rms(self.gated(emb_seq, hidden_seq), self.norm_conv)
        normed_b = self.rms(g_b, self.norm_conv)
        acc = np.zeros_like(normed_b)
        for k in range(self.taps):
            back = (self.taps - 1 - k) * self.dil
            w_k = self.conv1d[:, :, k]
            if t - back < 0:
                continue
            acc += (normed_b if back == 0 else normed_true[t - back][None]) * w_k[None]
        return (g_b + self._silu(acc)).astype(np.float32)

    def jacobian_out(self, emb_seq, hidden_seq, t: int, coords=None, step: float = 1e-3):
        emb_seq = np.asarray(emb_seq, dtype=np.float32)
        coords = np.arange(self.n) if coords is None else np.asarray(coords, dtype=np.int64)
        jac = np.empty((self.hc * self.n, coords.size), dtype=np.float64)
        for lo in range(0, coords.size, 512):
            idx = coords[lo:lo + 512]
            m = idx.size
            plus = np.tile(emb_seq[t], (m, 1)).astype(np.float32)
            minus = plus.copy()
            plus[np.arange(m), idx] += step
            minus[np.arange(m), idx] -= step
            out = self.ple_out_at(np.concatenate([plus, minus]), emb_seq, hidden_seq, t)
            d = out[:m].reshape(m, -1).astype(np.float64) - out[m:].reshape(m, -1).astype(np.float64)
            jac[:, lo:lo + m] = (d / (2.0 * step)).T
        return jac


def ple_out_numpy(emb, hidden, w: dict, hc: int, n_embd: int, eps: float, dilation: int = 3) -> np.ndarray:
    """``hidden + PleReplica.ple_out(emb, hidden)`` over a whole sequence
    (zero history): the sum ``qwen4exp.cpp build_ple`` forms
    (``tests/test_replica_layers.py:247-250``)."""
    r = Replica(w, hc, n_embd, eps, dilation)
    return (np.asarray(hidden, dtype=np.float32) + r.ple_out(emb, hidden)).astype(np.float32)
