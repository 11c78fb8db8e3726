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


def _replica(hc=4, n=256, seed=0, conv_zero=False):
    w = {k: v.numpy() for k, v in ple_weights(hc, n, seed=seed).items()}
    r = P.Replica(w, hc, n, 1e-6, 3)
    if conv_zero:
        r.conv1d[:] = 0.0
    return r


def _seq(t_len, hc, n, seed):
    rng = np.random.default_rng(seed)
    emb = rng.standard_normal((t_len, n)).astype(np.float32)
    emb = emb / np.linalg.norm(emb, axis=1, keepdims=True) * 0.1
    return emb, rng.standard_normal((t_len, hc, n)).astype(np.float32)


def test_replica_known_answers():
    """The reference's PleReplica known answers (tests/test_lens.py:210-290),
    on random weights of a smaller width."""
    r = _replica()
    hc, n = 4, 256
    # a zero embedding: gate exactly 1/2, gated exactly 0
    hidden = np.random.default_rng(1).standard_normal((3, hc, n)).astype(np.float32)
    emb0 = np.zeros((3, n), dtype=np.float32)
    np.testing.assert_array_equal(r.gate(emb0, hidden), np.full((3, hc), 0.5, dtype=np.float32))
    assert np.all(r.gated(emb0, hidden) == 0.0)
    # the gate is scale invariant in emb, gated linear
    rng = np.random.default_rng(2)
    emb = rng.standard_normal((5, n)).astype(np.float32)  # unit-scale: eps is negligible
    hidden = rng.standard_normal((5, hc, n)).astype(np.float32)
    np.testing.assert_allclose(r.gate(emb, hidden), r.gate(emb * 10.0, hidden), atol=1e-6)
    np.testing.assert_allclose(r.gated(emb * 10.0, hidden), r.gated(emb, hidden) * 10.0, rtol=1e-4, atol=1e-5)
    # one position: only the last tap reads a row
    g1 = np.random.default_rng(3).standard_normal((1, hc, n)).astype(np.float32)
    pre = r.rms(g1, r.norm_conv)[0] * r.conv1d[:, :, 3]
    np.testing.assert_allclose(r.conv_out(g1)[0], pre / (1.0 + np.exp(-pre)), rtol=1e-5, atol=1e-6)
    # ple_out = gated + conv_out(gated); ple_out_at at the true embedding = ple_out
    emb, hidden = _seq(12, hc, n, 10)
    out = r.ple_out(emb, hidden)
    g = r.gated(emb, hidden)
    np.testing.assert_array_equal(out, g + r.conv_out(g))
    for t in (11, 5, 0):
        np.testing.assert_allclose(r.ple_out_at(emb[t][None], emb, hidden, t)[0], out[t], rtol=1e-5, atol=1e-6)


def test_replica_jacobian_finite_differences_and_closed_form():
    """tests/test_lens.py:292-345: the Jacobian against an independent central
    difference of ple_out_at, and, with the convolution zeroed and a zero
    hidden state (gate 1/2), against 0.5 * w_value tiled over the streams."""
    hc, n = 4, 256
    r = _replica()
    emb, hidden = _seq(12, hc, n, 2)
    t = 7
    k = r.key(emb[t:t + 1])
    q = r.rms(hidden[t:t + 1], r.norm_query)
    s = np.sum(k * q, axis=-1) / np.sqrt(n)
    assert np.min(np.abs(s)) > 0.05  # away from the gate's kink at s = 0
    coords = np.random.default_rng(5).choice(n, size=6, replace=False)
    jac = r.jacobian_out(emb, hidden, t, coords=coords, step=1e-3)
    h = 2e-3
    for i, c in enumerate(coords):
        plus, minus = emb[t].copy(), emb[t].copy()
        plus[c] += h
        minus[c] -= h
        fd = (r.ple_out_at(plus[None], emb, hidden, t)[0].reshape(-1).astype(np.float64)
              - r.ple_out_at(minus[None], emb, hidden, t)[0].reshape(-1).astype(np.float64)) / (2 * h)
        assert np.linalg.norm(jac[:, i] - fd) / np.linalg.norm(fd) <= 1e-3
    z = _replica(conv_zero=True)
    emb, _ = _seq(5, hc, n, 13)
    coords = np.random.default_rng(6).choice(n, size=6, replace=False)
    jac = z.jacobian_out(emb, np.zeros((5, hc, n), dtype=np.float32), 2, coords=coords, step=1e-3)
    exp = np.tile(0.5 * z.w_value[:, coords], (hc, 1))
    assert np.linalg.norm(jac - exp) / np.linalg.norm(exp) <= 1e-3


def test_detached_gradients_sum_to_the_full_gradient():
    """layers.py:584-591: with detach_value the emb gradient flows through the
    gate only, with detach_gate through the value only; emb reaches the output
    only through gated = value * gate, so by the product rule the two add up to
    the undetached emb gradient.  (hidden and the history also reach the output
    directly, so for them the direct share would count twice.)"""
    hc, n, T = 4, 256, 14
    w = ple_weights(hc, n, seed=21)
    g = torch.Generator().manual_seed(22)
    emb = torch.randn((T, n), generator=g) * 0.1
    hidden = torch.randn((T, hc, n), generator=g) * 0.1
    hist = torch.randn((9, hc, n), generator=g) * 0.1
    r = torch.randn((T, hc, n), generator=g)
    grads = {}
    for dv, dg in ((False, False), (True, False), (False, True)):
        leaves = [x.clone().requires_grad_(True) for x in (emb, hidden, hist)]
        out, new_hist, _, _ = P.ple_forward(leaves[0], leaves[1], w, leaves[2], hc, n, 1e-6, 3,
                                            detach_value=dv, detach_gate=dg)
        ((out * r).sum() + new_hist.sum()).backward()
        grads[(dv, dg)] = [x.grad for x in leaves]
    full, a, b = grads[(False, False)][0], grads[(True, False)][0], grads[(False, True)][0]
    assert (a + b - full).abs().max().item() <= 1e-5 * full.abs().max().item()
    # the value path and the gate path each carry a share of the emb gradient
    assert grads[(True, False)][0].abs().max() > 0 and grads[(False, True)][0].abs().max() > 0
