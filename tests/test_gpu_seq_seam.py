"""The sequence seam on the GPU (engraft/replica/seq.py:570-637, 809-921,
1340-1470; the model's read at engraft/replica/model.py:845-853): a model
whose prefix loop reads every new position through ``replica.ple_true_emb``
runs under ``seq_forward`` / ``seq_step``, which shadow that method with
slices of the device ``OverlayEmb``.

Asserted, as the reference's step loop asserts and tests it
(tests/test_seq.py:33-46): ``n_ple_calls == n_prefix - start``; the patched
forward equals the unpatched one on the table's own rows (bit for bit); the
gradient that reaches ``rows_var`` equals the oracle's slot-ordered scatter of
d(loss)/d(emb) over the overlay's slots (the association of the descent
step); a packed sequence with segments and a prefix ``base_state``; the
instance attribute restored afterwards; a model that bypasses the method is
caught by the count check."""
from __future__ import annotations

import dataclasses
import sys

import numpy as np
import pytest
import torch

from oracle import backward as B
from oracle import overlay_emb as OE
from tests import gpu_util as G
from tests.params import fake_table_spec

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


@dataclasses.dataclass
class _State:
    n_prefix: int
    logits: torch.Tensor
    emb: torch.Tensor


class _Model:
    """A one-layer stand-in for ``Replica.prefix``: the PLE rows of the new
    positions are read one position at a time through ``self.ple_true_emb``
    (model.py:848), concatenated and moved to the device (model.py:853), then
    projected to logits.  Its own ``ple_true_emb`` reads the true rows."""

    def __init__(self, table, n_vocab: int, device, bypass: bool = False):
        from engraft_ngram_amd import seq
        self._seq = seq
        self.table = table
        self.bypass = bypass
        g = torch.Generator(device=device).manual_seed(7)
        self.w_out = (torch.randn((table.n_heads * table.row_len, n_vocab), generator=g, device=device) * 0.05).requires_grad_(True)
        self.device = device

    def ple_true_emb(self, tokens, t, overlay=None):
        return self._seq.ple_true_emb(self.table, tokens, t, overlay).cpu()

    def prefix(self, tokens, grad_proxy=True, return_logits=True, base_state=None, cache=None):
        start = base_state.n_prefix if base_state is not None else 0
        n_prefix = len(tokens) - 1
        read = type(self).ple_true_emb.__get__(self) if self.bypass else self.ple_true_emb
        rows = [read(tokens, t) for t in range(start, n_prefix)]
        emb = torch.cat(rows, dim=0).to(device=self.device, dtype=torch.float32)
        return _State(n_prefix=n_prefix, logits=emb @ self.w_out, emb=emb)


def test_seq_forward_and_step_through_the_patch(cuda):
    from engraft_ngram_amd import seq
    from engraft_ngram_amd.pack import pack_fragments
    _say("seq seam")
    spec = fake_table_spec(31, head_vocab_size=400)
    tab, fetch = G.f32_table(spec, 160, seed=32)
    rng = np.random.default_rng(33)
    frags = [[int(x) for x in rng.integers(0, 15, int(rng.integers(4, 60)))] for _ in range(12)]
    packed = pack_fragments(frags, spec.eos_token_id, max_len=400)[0]
    tokens = packed.tokens
    n_prefix = len(tokens) - 1
    seg = packed.segment_ids.numpy()
    rows, *_ = OE.build_plan(spec, tokens, {}, n_prefix, 0, seg)
    uniq = np.unique(rows)
    pick = np.sort(rng.choice(uniq, size=max(1, uniq.size // 4), replace=False))
    row_map = {int(g): i for i, g in enumerate(pick)}
    model = _Model(tab, n_vocab=97, device=cuda)
    # no overlay rows: the patched forward is the model's own forward
    empty = torch.zeros((0, 160), device=cuda, requires_grad=True)
    st0, stats0 = seq.seq_forward(model, tokens, empty, {}, segment_ids=packed.segment_ids)
    assert stats0.n_ple_calls == n_prefix and (stats0.n_id_hits, stats0.n_key_hits) == (0, 0)
    assert "ple_true_emb" not in model.__dict__
    plain = torch.cat([seq.ple_true_emb_range(tab, tokens, 0, n_prefix, seg_start=packed.seg_start())])
    assert torch.equal(st0.emb, plain)
    # a descent step through the patch, from position 0 and from a prefix state
    rv0 = (torch.randn((pick.size, 160), generator=torch.Generator().manual_seed(34)) * 0.05).to(cuda)
    c = torch.randn((n_prefix, 97), generator=torch.Generator().manual_seed(35)).to(cuda)
    for start in (0, 41):
        rv = rv0.clone().requires_grad_(True)
        base = _State(n_prefix=start, logits=None, emb=None) if start else None
        loss, timings, stats = seq.seq_step(model, tokens, rv, row_map, lambda s: (s.logits * c[start:]).sum(),
                                            base_state=base, segment_ids=packed.segment_ids)
        assert stats.n_ple_calls == n_prefix - start and stats.n_id_hits > 0
        assert set(timings) == {"fwd_s", "bwd_s", "pre_s"}
        assert "ple_true_emb" not in model.__dict__
        # d(loss)/d(emb) = c @ w_out^T; rows_var's gradient is its slot-ordered scatter
        d_emb = (c[start:] @ model.w_out.detach().T).cpu().numpy()
        _, (it, ih, ir), _, ni = OE.build(spec, tokens, row_map, rv0.cpu().numpy(), n_prefix, fetch, start=start,
                                          segment_ids=seg)
        assert ni == stats.n_id_hits
        grad, _ = B.scatter_grad_keys(d_emb, OE.slot_keys(it, ih, ir, n_prefix - start, 16), 16, pick.size)
        got = rv.grad.cpu().numpy()
        scale = np.maximum(np.abs(grad).max(axis=1, keepdims=True), 1e-30)
        assert float((np.abs(got - grad) / scale).max()) <= 1e-5


def test_seq_step_catches_a_patch_that_did_not_take(cuda):
    from engraft_ngram_amd import seq
    spec = fake_table_spec(36, head_vocab_size=200)
    tab, _ = G.f32_table(spec, 160, seed=37)
    tokens = [spec.eos_token_id, 3, 5, 7, 2, 9]
    model = _Model(tab, n_vocab=11, device=cuda, bypass=True)
    rv = torch.zeros((0, 160), device=cuda, requires_grad=True)
    with pytest.raises(AssertionError, match="n_ple_calls=0"):
        seq.seq_step(model, tokens, rv, {}, lambda s: s.logits.sum())
    assert "ple_true_emb" not in model.__dict__
