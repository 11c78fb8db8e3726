"""GPU parity of the sequence overlay (OverlayEmb), ple_true_emb, RowSet,
.pleo overlays and the damage scan against the oracle.

Bar: embeddings bit-exact (copies of dequantised / variable rows),
gradients bit-exact against the oracle's deterministic slot sum, hit counts
and ids exact, float statistics of the scan within 1e-6 relative."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import backward as B
from oracle import damage as DM
from oracle import hash as H
from oracle import overlay_emb as OE
from tests import gpu_util as G
from tests.params import fake_table_spec, reference_corpus, synthetic_spec

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).parent / "golden"


def _say(msg: str) -> None:
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


def _row_map(rows: np.ndarray, every: int, heads=(1, 6, 12)) -> dict:
    picked = set()
    for h in heads:
        picked |= set(rows[::every, h].tolist())
    return {g: i for i, g in enumerate(sorted(picked))}


def test_overlay_emb_int_keys_forward_and_grad(cuda):
    from engraft_ngram_amd.seq import OverlayEmb
    _say("OverlayEmb int keys, q8_0 table")
    spec = synthetic_spec(n_rows=16 * 700, seed=11)
    tab = G.device_table(spec, "q8_0", 16 * 700, 128, seed=12)
    fetch = G.synth_fetch("q8_0", 12, 128)
    tokens = [int(x) for x in np.random.default_rng(13).zipf(1.3, 600) % 900]
    rows = H.ngram_rows_np(spec, tokens)
    row_map = _row_map(rows, 5)
    R = len(row_map)
    rv = (torch.randn((R, 128), generator=torch.Generator().manual_seed(14)) * 0.05).to(cuda).requires_grad_(True)
    oe = OverlayEmb(tab, tokens, rv, row_map)
    emb = oe.build(600)
    exp, (it, ih, ir), nk, ni = OE.build(spec, tokens, row_map, rv.detach().cpu().numpy(), 600, fetch)
    assert np.array_equal(emb.detach().cpu().numpy(), exp)
    assert (oe.n_key_hits, oe.n_id_hits) == (nk, ni)
    d = torch.randn(emb.shape, generator=torch.Generator().manual_seed(15)).to(cuda)
    (emb * d).sum().backward()
    keys = OE.slot_keys(it, ih, ir, 600, 16)
    grad, hits = B.scatter_grad_keys(d.cpu().numpy(), keys, 16, R)
    assert hits.max() > B.PIECE  # a long segment was exercised
    assert np.array_equal(rv.grad.cpu().numpy(), grad)
    # a second build on the same instance with a reassigned rows_var reuses the plan
    oe.rows_var = torch.zeros_like(rv)
    e2 = oe.build(600).detach().cpu().numpy()
    exp2, *_ = OE.build(spec, tokens, row_map, np.zeros((R, 128), np.float32), 600, fetch)
    assert np.array_equal(e2, exp2)


def test_overlay_emb_long_keys_segments_and_start(cuda):
    from engraft_ngram_amd.pack import pack_fragments
    from engraft_ngram_amd.seq import OverlayEmb
    _say("OverlayEmb long keys + segments + start")
    spec = fake_table_spec(21, head_vocab_size=300)
    tab, fetch = G.f32_table(spec, 160, seed=22)
    rng = np.random.default_rng(23)
    frags = [[int(x) for x in rng.integers(0, 12, int(rng.integers(3, 40)))] for _ in range(30)]
    packed = pack_fragments(frags, spec.eos_token_id, max_len=512)[0]
    tokens = packed.tokens
    n = len(tokens) - 1
    seg = packed.segment_ids.numpy()
    rows, *_ = OE.build_plan(spec, tokens, {}, n, 0, seg)
    row_map = _row_map(rows, 9)
    R0 = len(row_map)
    for i, (w, h) in enumerate([((3, 4), 2), ((1, 1), 9), ((5, 7), 0), ((2, 2), 15)]):
        row_map[(w, h)] = R0 + i
    R = len(row_map)
    rv = (torch.randn((R, 160), generator=torch.Generator().manual_seed(24)) * 0.05).to(cuda).requires_grad_(True)
    for start in (0, 37):
        oe = OverlayEmb(tab, tokens, rv, row_map, segment_ids=packed.segment_ids)
        emb = oe.build(n, start=start)
        exp, (it, ih, ir), nk, ni = OE.build(spec, tokens, row_map, rv.detach().cpu().numpy(), n, fetch,
                                             start=start, segment_ids=seg)
        assert nk > 0 and ni > 0
        assert np.array_equal(emb.detach().cpu().numpy(), exp)
        assert (oe.n_key_hits, oe.n_id_hits) == (nk, ni)
        d = torch.randn(emb.shape, generator=torch.Generator().manual_seed(25 + start)).to(cuda)
        rv.grad = None
        (emb * d).sum().backward()
        grad, _ = B.scatter_grad_keys(d.cpu().numpy(), OE.slot_keys(it, ih, ir, n - start, 16), 16, R)
        assert np.array_equal(rv.grad.cpu().numpy(), grad)
    # the fragment cache gives the same embedding and counters, and is reused
    cache: dict = {}
    oe1 = OverlayEmb(tab, tokens, rv, row_map, segment_ids=packed.segment_ids, overlay_cache=cache)
    e1 = oe1.build(n).detach().cpu().numpy()
    oe0 = OverlayEmb(tab, tokens, rv, row_map, segment_ids=packed.segment_ids)
    assert np.array_equal(e1, oe0.build(n).detach().cpu().numpy())
    assert (oe1.n_key_hits, oe1.n_id_hits) == (oe0.n_key_hits, oe0.n_id_hits)
    n_entries = len(cache)
    assert n_entries > 0
    oe2 = OverlayEmb(tab, tokens, rv, row_map, segment_ids=packed.segment_ids, overlay_cache=cache)
    assert np.array_equal(oe2.build(n).detach().cpu().numpy(), e1) and len(cache) == n_entries


def test_ple_true_emb_and_rowset(cuda):
    """tests/test_replica_graft.py:43-70 on the device, and RowSet against
    the oracle's per-position re-hash."""
    from engraft_ngram_amd import lens, seq
    from engraft_ngram_amd.overlay import DeviceOverlay
    spec = fake_table_spec(7, head_vocab_size=500)
    tab, fetch = G.f32_table(spec, 160, seed=31)
    tokens = [1, 2, 3, 4, 5, spec.eos_token_id, 8, 9]
    for t in range(len(tokens)):
        rs = lens.RowSet.from_position(tab, tokens, t)
        r_exp, d_exp = OE.row_set(spec, tokens, t, fetch)
        assert np.array_equal(rs.rows_global, r_exp) and np.array_equal(rs.data, d_exp)
        plain = seq.ple_true_emb(tab, tokens, t).cpu().numpy()
        assert np.array_equal(plain, OE.ple_true_emb(spec, tokens, t, fetch))
    rs = lens.RowSet.from_position(tab, tokens, 3)
    vec = np.full(160, 99.0, np.float32)
    ov = {int(rs.rows_global[0]): vec}
    out = seq.ple_true_emb(tab, tokens, 3, overlay=ov).cpu().numpy().reshape(16, 160)
    assert np.array_equal(out[0], vec) and np.array_equal(out[1:], rs.data[1:])
    out2 = seq.ple_true_emb(tab, tokens, 3, overlay=DeviceOverlay.from_dict(ov, 160)).cpu().numpy()
    assert np.array_equal(out2.reshape(16, 160), out)
    rng_all = seq.ple_true_emb_range(tab, tokens, 0, len(tokens), overlay=ov).cpu().numpy()
    for t in range(len(tokens)):
        assert np.array_equal(rng_all[t:t + 1], OE.ple_true_emb(spec, tokens, t, fetch, ov))


def test_pleo_overlay_substitutes_real_rows(cuda):
    """The real .pleo fixtures as device overlays: gathering their own ids
    returns their vectors bit for bit (the substitution wins over the base
    table even where the id lies beyond a small base table)."""
    from engraft_ngram_amd import lens
    spec = fake_table_spec(3, head_vocab_size=100)
    tab, _ = G.f32_table(spec, 160, seed=41)
    for name in ("real_en_dog.pleo", "real_it_gatto.pleo"):
        rows, data = lens.read_pleo(GOLDEN / name)
        ov = lens.pleo_overlay(GOLDEN / name)
        got = tab.gather(torch.from_numpy(rows).reshape(-1, 1), overlay=ov).cpu().numpy()
        assert np.array_equal(got, data)


def test_scan_hits_against_oracle(cuda):
    """tests/test_damage.py:38-61's corpus and picks, device scan vs oracle."""
    from engraft_ngram_amd import damage
    _say("damage scan")
    spec = fake_table_spec(7)
    tab, _ = G.f32_table(spec, 32, seed=51)
    tokens = reference_corpus(20_000, seed=1, eos=spec.eos_token_id)
    rows = H.ngram_rows_np(spec, tokens)
    picks = [(100, 0), (150, 11), (300, 7), (777, 9), (5000, 5)]
    ov = np.array(sorted({int(rows[p, h]) for p, h in picks}), dtype=np.int64)
    dn = np.arange(1, ov.size + 1, dtype=np.float32) * 0.37
    big, tri = damage.ngram_rows(tokens, tab)
    assert np.array_equal(np.concatenate([big, tri], axis=1), rows)
    exp = DM.scan_hits(spec, tokens, ov, dn, block=4_000)
    for block in (4_000, 7_777, 20_000):
        got = damage.scan_hits(tokens, tab, ov, dn, block=block)
        for k in ("pos", "n_hit_rows", "dnorm_max", "read_count"):
            assert np.array_equal(got[k], exp[k]), k
        np.testing.assert_allclose(got["dnorm_sum"], exp["dnorm_sum"], rtol=1e-6)
