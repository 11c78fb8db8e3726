"""The CPU baselines the benchmark times beside the GPU legs, pinned against
the oracle: the threaded damage scan equals ``oracle.damage.scan_hits``; the
torch descent step (``index_add_`` + ``torch.optim.Adam`` + Q8_0) agrees with
the oracle's slot-ordered scatter and Adam step within the 1e-5 relative bar
and its requantisation with the oracle's rule."""
from __future__ import annotations

import numpy as np
import torch

from oracle import backward as B
from oracle import cpu_baseline as CB
from oracle import damage as OD
from oracle import formats as F
from oracle import hash as H
from tests.params import synthetic_spec


def test_threaded_scan_equals_oracle():
    spec = synthetic_spec(n_rows=16 * 5000, seed=3)
    rng = np.random.default_rng(1)
    tok = rng.integers(0, 300, size=60_000)
    tok[::777] = spec.eos_token_id
    ov = np.unique(rng.integers(0, 80_000, size=9000))
    dn = rng.random(ov.size).astype(np.float32)
    for threads in (1, 3, 8):
        r = CB.scan_block_threads(spec, tok, ov, dn, threads)
        o = OD.scan_hits(spec, tok, ov, dn, block=len(tok))
        pos = np.flatnonzero(r["n_hit"][:len(tok) - 1] > 0)
        assert np.array_equal(pos, o["pos"])
        assert np.array_equal(r["n_hit"][pos], o["n_hit_rows"])
        assert np.array_equal(r["dnorm_max"][pos], o["dnorm_max"])
        assert np.array_equal(r["dnorm_sum"][pos], o["dnorm_sum"])
        assert np.array_equal(r["read_count"], o["read_count"])


def test_torch_descent_step_matches_oracle():
    spec = synthetic_spec(n_rows=16 * 3000, seed=5)
    rng = np.random.default_rng(2)
    tok = rng.integers(0, 400, size=1500)
    rows = H.ngram_rows_np(spec, tok)
    ids = np.unique(rows)
    p0 = (rng.standard_normal((ids.size, 128)) * 0.02).astype(np.float32)
    d = (rng.standard_normal((tok.size, 16 * 128)) * 1e-3).astype(np.float32)
    td = CB.TorchDescent(torch.from_numpy(rows), torch.from_numpy(p0), lr=1e-3)
    assert np.array_equal(td.ids.numpy(), ids)
    q, dq = td.step(torch.from_numpy(d).to(torch.bfloat16))
    d_bf = torch.from_numpy(d).to(torch.bfloat16).float().numpy()
    grad, hits = B.scatter_grad(d_bf, rows, ids)
    p1, _, _ = B.adam_step(p0, grad, np.zeros_like(p0), np.zeros_like(p0), 1, 1e-3)
    got = td.param.detach().numpy()
    scale = np.maximum(np.abs(p1).max(axis=1, keepdims=True), 1e-30)
    assert float((np.abs(got - p1) / scale).max()) <= 1e-5
    eq, ed = F.quant_q8_0(got)
    assert np.array_equal(q.numpy(), eq) and np.array_equal(dq.numpy().view(np.uint16), ed.view(np.uint16))
