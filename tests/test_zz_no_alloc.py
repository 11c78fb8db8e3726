"""eg_descent_step_noalloc (the descent step whose grouping scratch is the
library's static per-GPU array) against eg_descent_step with a caller
workspace, through the C ABI: master rows, Adam moments and the requantised
rows bitwise equal after each of two steps in a row, the second on a smaller
batch (the static scratch then holds the first step's stale contents), and a
step too large for the static scratch refused before any launch."""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import hash as H
from oracle import synth
from tests import gpu_util as G
from tests.params import synthetic_spec

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


def _state_bits(st) -> list[np.ndarray]:
    out = [st.master.cpu().numpy().view(np.uint32), st.m.cpu().numpy().view(np.uint32),
           st.v.cpu().numpy().view(np.uint32), st.quant.payload.cpu().numpy().view(np.uint8)]
    if st.quant.scales is not None:
        out.append(st.quant.scales.cpu().numpy().view(np.uint8))
    return out


@pytest.mark.parametrize("fmt", ["q8_0", "mxfp8"])
def test_descent_step_noalloc_matches_workspace_form(cuda, fmt):
    from engraft_ngram_amd import _lib
    from engraft_ngram_amd import descent as D
    _say(f"noalloc descent step, {fmt}")
    spec = synthetic_spec(n_rows=16 * 6000, seed=91)
    tab = G.device_table(spec, fmt, 16 * 6000, 128, seed=92)
    big = synth.zipf_tokens(93, 4096, 3000)  # repeated bigrams: long segments
    small = synth.zipf_tokens(94, 700, 3000)
    rows_big = torch.from_numpy(H.ngram_rows_np(spec, big).astype(np.int32))
    rows_small = torch.from_numpy(H.ngram_rows_np(spec, small).astype(np.int32))
    every = torch.cat([rows_big.reshape(-1), rows_small.reshape(-1)])
    with_ws = D.DescentState.from_rows(tab, every, quant_fmt=fmt)
    no_ws = D.DescentState.from_rows(tab, every, quant_fmt=fmt)
    assert all(np.array_equal(a, b) for a, b in zip(_state_bits(with_ws), _state_bits(no_ws)))
    g = torch.Generator(device=cuda).manual_seed(95)
    for k, (rows, kw) in enumerate([(rows_big, {}), (rows_small, {"mu": 0.1})]):
        d = (torch.randn((rows.shape[0], 2048), generator=g, device=cuda) * 1e-3).to(torch.bfloat16)
        with_ws.step(d, rows, lr=1e-3, **kw)
        no_ws.step(d, rows, lr=1e-3, no_alloc=True, **kw)
        torch.cuda.synchronize()
        for name, a, b in zip(("master", "m", "v", "payload", "scales"), _state_bits(with_ws), _state_bits(no_ws)):
            assert np.array_equal(a, b), f"step {k}: {name} differs"
        _say(f"step {k} ({rows.shape[0]} positions) bitwise equal")
    assert _lib.load().eg_descent_step_noalloc_max_bytes() == 16 << 20


def test_descent_step_noalloc_refuses_oversize(cuda):
    from engraft_ngram_amd import _lib
    from engraft_ngram_amd import descent as D
    spec = synthetic_spec(n_rows=16 * 6000, seed=96)
    tab = G.device_table(spec, "q8_0", 16 * 6000, 128, seed=97)
    st = D.DescentState.from_rows(tab, torch.arange(0, 16 * 6000, 7, dtype=torch.int32))
    n_pos = 131072  # 2M slots: 24 MiB of scratch, more than the static 16 MiB
    need = _lib.load().eg_backward_workspace_size(n_pos * 16, st.n)
    assert need > _lib.load().eg_descent_step_noalloc_max_bytes()
    rows = torch.zeros((n_pos, 16), dtype=torch.int32, device=cuda)
    d = torch.zeros((n_pos, 2048), dtype=torch.bfloat16, device=cuda)
    before = st.master.clone()
    with pytest.raises(_lib.EgError, match="static"):
        st.step(d, rows, lr=1e-3, no_alloc=True)
    torch.cuda.synchronize()
    assert torch.equal(st.master, before) and st.step_count == 0
