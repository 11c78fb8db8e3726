"""The PLE block that consumes the gathered rows, on the device: the drop-in
for ``PleWeights`` / ``ple_forward`` (``engraft/replica/layers.py:555-626``).

Forward:

* ``key = emb @ w_key^T`` and ``value = emb @ w_value^T``: fp32 library GEMMs
  (hipBLASLt / rocBLAS through ``torch.matmul``, on the matrix cores);
* ``eg_ple_gate``: per position and stream, the RMS norms of key and hidden,
  the score ``s``, the gate, ``gated = value * gate`` and its RMS norm;
* ``eg_ple_conv``: the dilated causal depthwise convolution over
  ``[history; normed]``, SiLU, and ``out = hidden + gated + conv``.

The result -- the output and the new history -- is differentiable in emb,
hidden, the history and the weights.  The backward recomputes the block with
torch operations on the device and differentiates that; the forward values are
the HIP kernels'.  ``detach_value`` / ``detach_gate`` change only the backward,
as in the reference.
"""
from __future__ import annotations

import dataclasses

import torch
import torch.nn.functional as F

from . import _lib


@dataclasses.dataclass
class PleWeights:
    """``engraft/replica/layers.py:555-562``."""

    w_key: torch.Tensor  # [hc*n_embd, n_embd]
    w_value: torch.Tensor  # [n_embd, n_embd]
    norm_key: torch.Tensor  # [hc*n_embd]
    norm_query: torch.Tensor  # [hc*n_embd]
    norm_conv: torch.Tensor  # [hc*n_embd]
    conv1d: torch.Tensor  # [hc*n_embd, K]


def _rms(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    return x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + eps) * w


def _block_torch(emb, hidden, w_key, w_value, nk, nq, nc, conv, hist, eps, dil, detach_value, detach_gate):
    """The block in torch operations (the backward's recomputation): ``(out,
    new_hist)``."""
    t_len, hc, n = hidden.shape
    key = _rms((emb @ w_key.T).reshape(t_len, hc, n), nk.reshape(hc, n), eps)
    query = _rms(hidden, nq.reshape(hc, n), eps)
    s = (key * query).sum(dim=-1) / (n ** 0.5)
    gate = torch.sigmoid(torch.sign(s) * torch.sqrt(torch.clamp(s.abs(), min=1e-6)))
    value = emb @ w_value.T
    g = gate.detach() if detach_gate else gate
    v = value.detach() if detach_value else value
    gated = v.unsqueeze(1) * g.unsqueeze(-1)
    normed = _rms(gated, nc.reshape(hc, n), eps).reshape(t_len, hc * n)
    full = torch.cat([hist.reshape(hist.shape[0], hc * n), normed], dim=0)
    taps = conv.shape[1]
    h0 = hist.shape[0]
    acc = torch.zeros_like(normed)
    for k in range(taps):
        back = (taps - 1 - k) * dil
        lo = max(0, back - h0)  # first position whose source row exists
        if lo < t_len:
            acc[lo:] = acc[lo:] + full[h0 + lo - back:h0 + t_len - back] * conv[:, k]
    out = hidden + gated + F.silu(acc).reshape(t_len, hc, n)
    hist_len = (taps - 1) * dil
    new_hist = full[-hist_len:] if hist_len > 0 else full[:0]
    return out, new_hist.reshape(-1, hc, n)


class _PleFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, emb, hidden, w_key, w_value, nk, nq, nc, conv, hist, eps, dil, detach_value, detach_gate):
        t_len, hc, n = hidden.shape
        dev = hidden.device
        f32 = dict(dtype=torch.float32, device=dev)
        emb32 = emb.to(**f32).contiguous()
        key = (emb32 @ w_key.to(**f32).T).contiguous()
        value = (emb32 @ w_value.to(**f32).T).contiguous()
        hidden32 = hidden.to(**f32).contiguous()
        h0 = hist.shape[0]
        full = torch.empty((h0 + t_len, hc * n), **f32)
        if h0:
            full[:h0] = hist.reshape(h0, hc * n)
        s = torch.empty((t_len, hc), **f32)
        gate = torch.empty((t_len, hc), **f32)
        st = _lib.stream_ptr(dev)
        nk32, nq32, nc32 = (x.to(**f32).contiguous() for x in (nk, nq, nc))
        conv32 = conv.to(**f32).contiguous()
        _lib.call("eg_ple_gate", _lib.ptr(key), _lib.ptr(value), _lib.ptr(hidden32), _lib.ptr(nk32), _lib.ptr(nq32),
                  _lib.ptr(nc32), t_len, hc, n, float(eps), _lib.ptr(full[h0:]), _lib.ptr(s), _lib.ptr(gate), st)
        out = torch.empty((t_len, hc, n), **f32)
        _lib.call("eg_ple_conv", _lib.ptr(full), h0, t_len, hc, n, _lib.ptr(conv32), conv32.shape[1], int(dil),
                  _lib.ptr(hidden32), _lib.ptr(value), _lib.ptr(gate), _lib.ptr(out), st)
        hist_len = (conv32.shape[1] - 1) * int(dil)
        new_hist = (full[-hist_len:] if hist_len > 0 else full[:0]).reshape(-1, hc, n).to(hidden.dtype).clone()
        ctx.save_for_backward(emb, hidden, w_key, w_value, nk, nq, nc, conv, hist)
        ctx.cfg = (eps, dil, detach_value, detach_gate)
        ctx.mark_non_differentiable(s, gate, value)
        return out.to(hidden.dtype), new_hist, s, gate, value

    @staticmethod
    def backward(ctx, d_out, d_hist, _d_s, _d_gate, _d_value):
        inputs = ctx.saved_tensors
        eps, dil, detach_value, detach_gate = ctx.cfg
        with torch.enable_grad():
            leaves = [x.detach().requires_grad_(need) for x, need in zip(inputs, ctx.needs_input_grad[:9])]
            out, new_hist = _block_torch(*leaves, eps, dil, detach_value, detach_gate)
            wrt = [x for x, need in zip(leaves, ctx.needs_input_grad[:9]) if need]
            outs, grads_in = [out], [d_out]
            if d_hist is not None and new_hist.numel():
                outs.append(new_hist)
                grads_in.append(d_hist)
            grads = iter(torch.autograd.grad(outs, wrt, grads_in, allow_unused=True) if wrt else [])
        res = []
        for x, need in zip(leaves, ctx.needs_input_grad[:9]):
            g = next(grads) if need else None
            res.append(torch.zeros_like(x) if (need and g is None) else g)
        return (*res, None, None, None, None)


def ple_forward(emb: torch.Tensor, hidden: torch.Tensor, w: PleWeights, hist: torch.Tensor, hparams,
                diag: dict | None = None, detach_value: bool = False,
                detach_gate: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """``(hidden + gated + conv_out, new history)`` (``engraft/replica/layers.py:
    565-626``).  ``emb [T, n_embd]``, ``hidden [T, hc, n_embd]``, ``hist``
    ``[rows, hc, n_embd]`` (at most ``(K-1)*ple_ngram_size`` rows, empty at a
    sequence start); all on the device."""
    hc = hparams.hc_mult
    n = hparams.n_embd
    eps = float(hparams.f_norm_rms_eps)
    dil = int(hparams.ple_ngram_size)
    if hidden.dim() != 3 or hidden.shape[1:] != (hc, n) or emb.shape != (hidden.shape[0], n):
        raise ValueError(f"emb [T, {n}] and hidden [T, {hc}, {n}] expected, got {tuple(emb.shape)}, "
                         f"{tuple(hidden.shape)}")
    hist = hist.reshape(-1, hc, n) if hist.numel() else hidden.new_zeros((0, hc, n))
    out, new_hist, s, gate, value = _PleFn.apply(emb, hidden, w.w_key, w.w_value, w.norm_key, w.norm_query,
                                                 w.norm_conv, w.conv1d, hist, eps, dil, detach_value, detach_gate)
    if diag is not None:
        gated_norm = value.norm(dim=-1, keepdim=True) * gate.abs()
        diag["s"] = s.clone()
        diag["gate"] = gate.clone()
        diag["value_norm"] = value.norm(dim=-1).clone()
        diag["gated_norm"] = gated_norm.clone()
        diag["hidden_norm"] = hidden.detach().norm(dim=-1).clone()
    return out, new_hist
