"""Oracle: the PLE block that consumes the gathered rows (TEST
INFRASTRUCTURE ONLY -- see oracle/__init__.py).

* ``ple_forward``  -- torch fp32 on the CPU, step for step as
  ``engraft/replica/layers.py:565-626`` with ``rmsnorm`` (``:22-35``),
  ``rmsnorm_grouped`` (``:37-42``) and the per-position loop of
  ``causal_depthwise_conv`` (``:257-293``).
* ``ple_out_numpy`` -- the independent numpy formulation of the same block
  (``PleReplica`` in ``engraft/lens.py:221-341``: fp64 mean of squares, the
  shifted-array convolution with a fixed dilation).

Pinning (tests/test_oracle_ple.py): the two agree within 1e-4 on the real
dimensions (hc 4, n_embd 2560, 4 taps, dilation 3), per position with the
returned history as on the whole sequence, as the reference's own
``tests/test_replica_layers.py:238-282`` checks them.
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


def ple_forward(emb, hidden, w: dict, hist, hc: int, n_embd: int, eps: float, ngram_size: int):
    """Returns ``(out [T, hc, n], new_hist, s [T, hc], gate [T, hc])``."""
    t_len = emb.shape[0]
    key = (emb @ w["w_key"].T).reshape(t_len, hc, n_embd)
    key = rmsnorm_grouped(key, w["norm_key"], eps, hc)
    query = rmsnorm_grouped(hidden, w["norm_query"], eps, hc)
    s = (key * query).sum(dim=-1) / (n_embd ** 0.5)
    mag = torch.sqrt(torch.clamp(s.abs(), min=1e-6))
    gate = torch.sigmoid(torch.sign(s) * mag)
    value = emb @ w["w_value"].T
    gated = value.unsqueeze(1) * gate.unsqueeze(-1)
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


def ple_out_numpy(emb, hidden, w: dict, hc: int, n_embd: int, eps: float, dilation: int = 3) -> np.ndarray:
    """``hidden + PleReplica.ple_out(emb, hidden)`` over a whole sequence
    (zero history)."""
    def rms(x, weight):
        ms = np.mean(x.astype(np.float64) ** 2, axis=-1, keepdims=True)
        return (x / np.sqrt(ms + eps)).astype(np.float32) * weight

    nk = np.asarray(w["norm_key"]).reshape(hc, n_embd)
    nq = np.asarray(w["norm_query"]).reshape(hc, n_embd)
    nc = np.asarray(w["norm_conv"]).reshape(hc, n_embd)
    taps = np.asarray(w["conv1d"]).shape[1]
    conv = np.asarray(w["conv1d"]).reshape(hc, n_embd, taps)
    k = rms((emb @ np.asarray(w["w_key"]).T).reshape(-1, hc, n_embd), nk)
    q = rms(hidden, nq)
    s = (np.sum(k * q, axis=-1) / np.sqrt(n_embd)).astype(np.float64)
    gate = (1.0 / (1.0 + np.exp(-(np.sign(s) * np.sqrt(np.clip(np.abs(s), 1e-6, None)))))).astype(np.float32)
    v = (emb @ np.asarray(w["w_value"]).T).astype(np.float32)
    gated = (v[:, None, :] * gate[:, :, None]).astype(np.float32)
    normed = rms(gated, nc)
    t_len = normed.shape[0]
    acc = np.zeros_like(normed)
    for kk in range(taps):
        back = (taps - 1 - kk) * dilation
        w_k = conv[:, :, kk]
        if back == 0:
            acc += normed * w_k[None]
        elif back < t_len:
            sh = np.zeros_like(normed)
            sh[back:] = normed[:t_len - back]
            acc += sh * w_k[None]
    conv_out = (acc / (1.0 + np.exp(-acc))).astype(np.float32)
    return (hidden + gated + conv_out).astype(np.float32)
