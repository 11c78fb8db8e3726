"""GPU parity of PleReplica (engraft/lens.py:221-415) on the HIP kernels
against the numpy oracle ``oracle.ple.Replica`` at the real dimensions (hc 4,
n_embd 2560, 4 taps, dilation 3), plus the reference's known answers
(tests/test_lens.py:210-345) and the weights read from a model GGUF.

Bar (floating point, the reference's own): values within 1e-4 of the oracle;
the identities the reference asserts exactly (ple_out = gated + conv_out,
gate 1/2 at a zero embedding) hold bit for bit; the Jacobian within 1e-3
relative of its closed form / of a finite difference."""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import ple as P
from tests import gguf_util as GU
from tests.test_oracle_ple import ple_weights

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


def _pair(hc=4, n=2560, seed=3, device="cuda:0"):
    from engraft_ngram_amd.ple import PleReplica, PleWeights
    w = ple_weights(hc, n, seed=seed)
    dev = PleReplica.from_weights(PleWeights(**w), 1e-6, hc=hc, device=device)
    ref = P.Replica({k: v.numpy() for k, v in w.items()}, hc, n, 1e-6, 3)
    return dev, ref


def _seq(t_len, hc, n, seed, norm=0.1):
    rng = np.random.default_rng(seed)
    emb = rng.standard_normal((t_len, n)).astype(np.float32)
    emb = emb / np.linalg.norm(emb, axis=1, keepdims=True) * norm
    return emb, rng.standard_normal((t_len, hc, n)).astype(np.float32)


def _close(got: torch.Tensor, exp: np.ndarray, atol: float = 1e-4) -> None:
    g = got.cpu().numpy()
    assert g.shape == exp.shape
    err = float(np.abs(g - exp).max())
    assert err <= atol, f"max |diff| {err}"


def test_ple_replica_methods_against_oracle(cuda):
    _say("PleReplica methods, hc 4 x 2560")
    dev, ref = _pair(device=cuda)
    emb, hidden = _seq(12, 4, 2560, 10)
    _close(dev.key(emb), ref.key(emb))
    _close(dev.value(emb), ref.value(emb))
    _close(dev.gate(emb, hidden), ref.gate(emb, hidden))
    _close(dev.gated(emb, hidden), ref.gated(emb, hidden))
    g = ref.gated(emb, hidden)
    _close(dev.conv_out(g), ref.conv_out(g))
    out = dev.ple_out(emb, hidden)
    _close(out, ref.ple_out(emb, hidden))
    # the reference's exact identity (tests/test_lens.py:275-285)
    gd = dev.gated(emb, hidden)
    assert torch.equal(out, gd + dev.conv_out(gd))
    # one-token continuations: the true embedding gives ple_out[t] bit for bit
    rng = np.random.default_rng(11)
    for t in (11, 5, 0):
        batch = np.concatenate([emb[t][None], rng.standard_normal((2, 2560)).astype(np.float32) * 0.003])
        at = dev.ple_out_at(batch, emb, hidden, t)
        _close(at, ref.ple_out_at(batch, emb, hidden, t))
        assert torch.equal(at[0], out[t])


def test_ple_replica_known_answers(cuda):
    _say("PleReplica known answers")
    dev, _ = _pair(device=cuda)
    hidden = np.random.default_rng(1).standard_normal((3, 4, 2560)).astype(np.float32)
    emb0 = np.zeros((3, 2560), dtype=np.float32)
    assert torch.equal(dev.gate(emb0, hidden).cpu(), torch.full((3, 4), 0.5))
    assert bool((dev.gated(emb0, hidden) == 0).all())
    # one position: only the last tap reads a row (tests/test_lens.py:238-251)
    g1 = np.random.default_rng(3).standard_normal((1, 4, 2560)).astype(np.float32)
    _, ref = _pair(device=cuda)
    pre = ref.rms(g1, ref.norm_conv)[0] * ref.conv1d[:, :, 3]
    _close(dev.conv_out(g1)[0], pre / (1.0 + np.exp(-pre)), atol=1e-5)


def test_ple_replica_jacobian(cuda):
    """Closed form with the convolution zeroed and zero hidden state
    (tests/test_lens.py:321-345), and a finite difference of ple_out_at at a
    second step size (tests/test_lens.py:288-319)."""
    _say("PleReplica jacobian")
    dev, ref = _pair(device=cuda)
    rng = np.random.default_rng(2)
    # rows of norm 1: the central differences resolve the derivative in fp32 (at
    # norm 0.1 the key's RMS norm bends within a step of 1e-3)
    emb, hidden = _seq(12, 4, 2560, 2, norm=1.0)
    t = 7
    coords = rng.choice(2560, size=8, replace=False)
    jac = dev.jacobian_out(emb, hidden, t, coords=coords, step=1e-3).cpu().numpy()
    assert jac.shape == (4 * 2560, 8)
    h = 2e-3
    for i, c in enumerate(coords):
        plus, minus = emb[t].copy(), emb[t].copy()
        plus[c] += h
        minus[c] -= h
        fd = (dev.ple_out_at(plus[None], emb, hidden, t)[0].reshape(-1).double()
              - dev.ple_out_at(minus[None], emb, hidden, t)[0].reshape(-1).double()).cpu().numpy() / (2 * h)
        assert np.linalg.norm(jac[:, i] - fd) / np.linalg.norm(fd) <= 1e-3
    dev.conv1d.zero_()
    emb, _ = _seq(5, 4, 2560, 13)
    coords = rng.choice(2560, size=6, replace=False)
    jac = dev.jacobian_out(emb, np.zeros((5, 4, 2560), dtype=np.float32), 2, coords=coords).cpu().numpy()
    exp = np.tile(0.5 * ref.w_value[:, coords], (4, 1))
    assert np.linalg.norm(jac - exp) / np.linalg.norm(exp) <= 1e-3


def test_ple_replica_from_gguf(cuda, tmp_path):
    """The weights of a split model GGUF (Q8_0 projections, F32 norms and taps,
    eps in shard 1) read to their closed-form values, and the block on them."""
    from engraft_ngram_amd.ple import PleReplica
    _say("PleReplica from a GGUF")
    hc, n = 4, 256
    w = {k: v.numpy() for k, v in ple_weights(hc, n, seed=5).items()}
    path, vals = GU.ple_model_files(tmp_path, w, 1e-5)
    dev = PleReplica(path, device=cuda)
    assert dev.eps == float(np.float32(1e-5))
    assert np.array_equal(dev.w_key.cpu().numpy(), vals["w_key"])
    assert np.array_equal(dev.w_value.cpu().numpy(), vals["w_value"])
    assert np.array_equal(dev.conv1d.cpu().numpy(), vals["conv1d"].reshape(hc, n, 4))
    ref = P.Replica(vals, hc, n, dev.eps, 3)
    emb, hidden = _seq(9, hc, n, 6)
    _close(dev.ple_out(emb, hidden), ref.ple_out(emb, hidden))
    with pytest.raises(ValueError):
        PleReplica(path, device=cuda, hc=2)  # the tensors do not have 2 streams
