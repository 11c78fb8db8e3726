"""Host logic of the sequence seam (no GPU): ``ple_emb_patched`` shadows
``replica.ple_true_emb`` with slices of the precomputed embedding at
``t - start``, counts the calls, and restores the instance exactly as it was
(attribute absent, or a previous instance attribute), on exit and on an
exception (engraft/replica/seq.py:570-637); ``seq_forward`` refuses fewer
than two tokens (engraft/replica/seq.py:892-893)."""
from __future__ import annotations

import pytest
import torch


class _Replica:
    def ple_true_emb(self, tokens, t, overlay=None):
        return torch.full((1, 4), -1.0)


def test_patch_slices_counts_and_restores():
    from engraft_ngram_amd import seq
    r = _Replica()
    emb = torch.arange(20.0).reshape(5, 4)
    stats = seq.PatchStats()
    with seq.ple_emb_patched(r, emb, stats, start=3):
        got = torch.cat([r.ple_true_emb([0] * 9, t) for t in range(3, 8)])
    assert torch.equal(got, emb) and stats.n_ple_calls == 5
    assert "ple_true_emb" not in r.__dict__
    assert torch.equal(r.ple_true_emb([0], 0), torch.full((1, 4), -1.0))
    # a previous instance attribute comes back, also after an exception
    mine = lambda tokens, t, overlay=None: "mine"  # noqa: E731
    r.ple_true_emb = mine
    with pytest.raises(RuntimeError):
        with seq.ple_emb_patched(r, emb, seq.PatchStats()):
            assert r.ple_true_emb([0], 2).shape == (1, 4)
            raise RuntimeError("inside")
    assert r.__dict__["ple_true_emb"] is mine


def test_seq_forward_needs_two_tokens():
    from engraft_ngram_amd import seq
    with pytest.raises(ValueError):
        seq.seq_forward(_Replica(), [5], torch.zeros(0, 4), {})
    with pytest.raises(ValueError):
        seq.seq_step(_Replica(), [5], torch.zeros(0, 4), {}, lambda s: s)
