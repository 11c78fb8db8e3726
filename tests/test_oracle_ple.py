"""Pins of the PLE block oracle (CPU): the torch restatement of ple_forward
against the independent numpy formulation, as the reference's own
tests/test_replica_layers.py:238-282 compares them."""
from __future__ import annotations

import numpy as np
import torch

from oracle import ple as P


def ple_weights(hc: int, n: int, taps: int = 4, seed: int = 0) -> dict:
    rng = np.random.default_rng(seed)
    f = lambda *s, sc=1.0: torch.from_numpy((rng.standard_normal(s) * sc).astype(np.float32))
    return {"w_key": f(hc * n, n, sc=n ** -0.5), "w_value": f(n, n, sc=n ** -0.5),
            "norm_key": 1.0 + f(hc * n, sc=0.1), "norm_query": 1.0 + f(hc * n, sc=0.1),
            "norm_conv": 1.0 + f(hc * n, sc=0.1), "conv1d": f(hc * n, taps, sc=0.5)}


def test_ple_torch_matches_numpy_replica_per_position():
    hc, n, T = 4, 2560, 5
    w = ple_weights(hc, n)
    emb = np.random.default_rng(1).standard_normal((T, n)).astype(np.float32) * 0.1
    hidden = np.random.default_rng(2).standard_normal((T, hc, n)).astype(np.float32) * 0.1
    ref = P.ple_out_numpy(emb, hidden, {k: v.numpy() for k, v in w.items()}, hc, n, 1e-6, dilation=3)
    hist = torch.zeros(0, hc, n)
    outs = []
    for t in range(T):
        out, hist, _, _ = P.ple_forward(torch.from_numpy(emb[t:t + 1]), torch.from_numpy(hidden[t:t + 1]), w, hist,
                                        hc, n, 1e-6, 3)
        outs.append(out[0].numpy())
    assert np.abs(np.stack(outs) - ref).max() < 1e-4
    # the whole sequence at once equals the per-position chain (history carried)
    out_all, hist_all, _, _ = P.ple_forward(torch.from_numpy(emb), torch.from_numpy(hidden), w, torch.zeros(0, hc, n),
                                            hc, n, 1e-6, 3)
    np.testing.assert_allclose(out_all.numpy(), np.stack(outs), atol=1e-5)
    assert torch.allclose(hist_all, hist, atol=1e-6)
    assert hist_all.shape[0] == min(T, 9)
