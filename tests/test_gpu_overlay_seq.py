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


def test_overlay_emb_backward_is_the_native_function(cuda):
    """build() returns the C++ autograd function's output (its backward takes
    no GIL); an upstream gradient in bf16 (which autograd casts to the output's
    f32) gives the gradient of its f32 copy; bf16 variables give a bf16
    embedding and the f32 gradient rounded once; host variables give a host
    embedding and gradient; a forward without a gradient makes no slot
    grouping."""
    from engraft_ngram_amd.seq import OverlayEmb
    _say("OverlayEmb native autograd node, bf16 gradient")
    spec = synthetic_spec(n_rows=16 * 700, seed=41)
    tab = G.device_table(spec, "q8_0", 16 * 700, 128, seed=42)
    tokens = [int(x) for x in np.random.default_rng(43).zipf(1.3, 300) % 900]
    rows = H.ngram_rows_np(spec, tokens)
    row_map = _row_map(rows, 4)
    R = len(row_map)
    rv = (torch.randn((R, 128), generator=torch.Generator().manual_seed(44)) * 0.05).to(cuda)
    oe = OverlayEmb(tab, tokens, rv, row_map)
    with torch.no_grad():
        oe.build(300)
    assert "grouping" not in oe._plans[(0, 300)]
    rv.requires_grad_(True)
    emb = oe.build(300)
    assert "GatherSlots" in emb.grad_fn.name()
    d = torch.randn(emb.shape, generator=torch.Generator().manual_seed(45)).to(cuda).bfloat16()
    emb.backward(d)
    g32 = rv.grad.clone()
    rv.grad = None
    oe.build(300).backward(d.float())
    assert torch.equal(g32, rv.grad)
    rvb = rv.detach().bfloat16().requires_grad_(True)
    oe.rows_var = rvb
    eb = oe.build(300)
    assert eb.dtype == torch.bfloat16
    assert torch.equal(eb.float(), oe.build(300).detach().float())
    eb.backward(d)
    assert rvb.grad.dtype == torch.bfloat16 and torch.equal(rvb.grad, g32.bfloat16())
    # variables on the host: the embedding comes back there, the gradient too
    rvc = rv.detach().cpu().requires_grad_(True)
    oe.rows_var = rvc
    ec = oe.build(300)
    assert ec.device.type == "cpu" and torch.equal(ec.detach(), emb.detach().cpu())
    ec.backward(d.float().cpu())
    assert rvc.grad.device.type == "cpu" and torch.equal(rvc.grad, g32.cpu())


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
    # the same as a method of a model class that keeps its table in self.table

    class Model(seq.ReplicaTableMixin):
        def __init__(self, table):
            self.table = table

    m = Model(tab)
    for t in (0, 3, len(tokens) - 1):
        assert torch.equal(m.ple_true_emb(tokens, t, overlay=ov), seq.ple_true_emb(tab, tokens, t, overlay=ov))


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
        for toks in (tokens, np.asarray(tokens, dtype=np.int32)):  # int64 and int32 token arrays
            got = damage.scan_hits(toks, tab, ov, dn, block=block)
            for k in ("pos", "n_hit_rows", "dnorm_max", "read_count"):
                assert np.array_equal(got[k], exp[k]), k
            np.testing.assert_allclose(got["dnorm_sum"], exp["dnorm_sum"], rtol=1e-6)


def test_scan_hits_edges_against_oracle(cuda):
    """Corpora shorter than the n-gram history, one block of exactly the
    history, every position in its own block, an empty and a one-row overlay,
    EOS runs; device scan vs oracle, and blocks below the history refused."""
    from engraft_ngram_amd import damage
    _say("damage scan edges")
    spec = fake_table_spec(7)
    tab, _ = G.f32_table(spec, 32, seed=52)
    hist = spec.ngram_size - 1
    corpus = reference_corpus(600, seed=3, eos=spec.eos_token_id)
    corpus[40:45] = spec.eos_token_id
    rows = H.ngram_rows_np(spec, corpus)
    overlays = [np.zeros(0, dtype=np.int64), np.array([rows[7, 3]], dtype=np.int64),
                np.unique(rows[::37].reshape(-1))]
    for n_tok in (0, 1, 2, 3, 4, 600):
        toks = corpus[:n_tok]
        for ov in overlays:
            dn = np.linspace(0.5, 2.0, ov.size).astype(np.float32)
            for block in sorted({hist, 5, 600}):
                exp = DM.scan_hits(spec, toks, ov, dn, block=block)
                got = damage.scan_hits(toks, tab, ov, dn, block=block)
                for k in ("pos", "n_hit_rows", "dnorm_max", "read_count"):
                    assert np.array_equal(got[k], exp[k]), (n_tok, ov.size, block, k)
                np.testing.assert_allclose(got["dnorm_sum"], exp["dnorm_sum"], rtol=1e-6)
    with pytest.raises(ValueError, match="history"):
        damage.scan_hits(corpus, tab, overlays[1], np.ones(1, np.float32), block=hist - 1)


def _mix32(x: int) -> int:
    m = 0xFFFFFFFF
    x &= m
    x ^= x >> 16
    x = (x * 0x7FEB352D) & m
    x ^= x >> 15
    x = (x * 0x846CA68B) & m
    return x ^ (x >> 16)


def _bloom_probe(row: int, n_fb: int) -> tuple[int, int]:
    """The filter block and bits of a row in eg_build_id_bitmap's blocked
    Bloom filter (the library's hash, restated to check the built blocks)."""
    x = _mix32(row)
    y = _mix32(x ^ 0x9E3779B9)
    mask = 0
    for sh in (0, 6, 12, 18, 24):
        mask |= 1 << ((y >> sh) & 63)
    return (x * n_fb) >> 32, mask


def test_scan_overlay_rank_bitmap(cuda):
    """eg_scan_overlay with and without the eg_build_id_bitmap rank bitmap:
    the pairs' bits hold exactly the ids below n_bits (an id past the table's
    rows is left out and still never hits), their ranks are the lower bounds
    of 32 w in the ids, every id's three filter bits are set in its filter
    word and the filter holds no other bit, and both launches give the same
    per-position outputs and read counts (bit-exact)."""
    import ctypes

    from engraft_ngram_amd import _lib
    _say("scan rank bitmap")
    spec = fake_table_spec(7)
    tab, _ = G.f32_table(spec, 32, seed=52)
    tokens = reference_corpus(30_000, seed=3, eos=spec.eos_token_id)
    rows = H.ngram_rows_np(spec, tokens)
    rng = np.random.default_rng(53)
    n_bits = tab.n_rows
    picked = set(rows[rng.integers(0, len(tokens), 40), rng.integers(0, rows.shape[1], 40)].tolist())
    picked |= set(rng.integers(0, n_bits, 3000).tolist()) | {0, n_bits - 1, n_bits + 5}
    ov = np.array(sorted(picked), dtype=np.int32)
    ids = torch.from_numpy(ov).to(cuda)
    dn = torch.from_numpy(rng.random(ov.size).astype(np.float32)).to(cuda)
    nw = (n_bits + 31) // 32
    n_fb = (nw + 63) // 64
    assert _lib.load().eg_id_bitmap_words(n_bits) == 2 * nw + 2 * n_fb
    bitmap = torch.full((2 * nw + 2 * n_fb,), -1, dtype=torch.int32, device=cuda)  # stale bits get cleared
    _lib.call("eg_build_id_bitmap", _lib.ptr(ids), ov.size, _lib.ptr(bitmap), n_bits, _lib.stream_ptr(cuda))
    want = np.zeros(nw * 32, dtype=bool)
    want[ov[ov < n_bits]] = True
    bm = bitmap.cpu().numpy()
    got_bits = np.unpackbits(bm[0:2 * nw:2].copy().view(np.uint8), bitorder="little").astype(bool)
    assert np.array_equal(got_bits, want)
    assert np.array_equal(bm[1:2 * nw:2].astype(np.int64), np.searchsorted(ov, np.arange(nw, dtype=np.int64) * 32))
    filt = bm[2 * nw:].copy().view(np.uint64)
    want_f = np.zeros(n_fb, dtype=np.uint64)
    for r in ov[ov < n_bits].tolist():
        b, mask = _bloom_probe(r, n_fb)
        want_f[b] |= np.uint64(mask)
    assert np.array_equal(filt, want_f)
    assert filt.any()
    tok = torch.from_numpy(np.asarray(tokens, dtype=np.int64)).to(cuda)
    spec_c = tab.c_spec
    outs = []
    for start in (0, 2):
        for bm in (None, _lib.ptr(bitmap)):
            m = tok.numel() - start
            n_hit = torch.empty(m, dtype=torch.int32, device=cuda)
            dmax, dsum = torch.empty(m, device=cuda), torch.empty(m, device=cuda)
            counts = torch.zeros(ov.size, dtype=torch.int64, device=cuda)
            _lib.call("eg_scan_overlay", ctypes.byref(spec_c), _lib.ptr(tok), 8, tok.numel(), start, _lib.ptr(ids),
                      ov.size, bm, n_bits, _lib.ptr(dn), _lib.ptr(n_hit), _lib.ptr(dmax), _lib.ptr(dsum),
                      _lib.ptr(counts), _lib.stream_ptr(cuda))
            outs.append([x.cpu().numpy() for x in (n_hit, dmax, dsum, counts)])
        for a, b in zip(outs[-2], outs[-1]):
            assert np.array_equal(a, b)
    assert int(outs[0][0].sum()) > 0 and int(outs[0][3][-1]) == 0


@pytest.mark.parametrize("n_files", [4, 40])
def test_sum_overlays_against_oracle(cuda, tmp_path, n_files):
    """engraft/replica/overlay_sum.py:38-112 on the device: the union, the
    merged rows bit-exact against the reference's order (each row's deltas
    added one at a time, file after file; 40 files put 40 deltas on a row,
    one file lists a row twice) and the manifest; write_merged_pleo's order."""
    from engraft_ngram_amd import lens, overlay_sum
    from oracle import overlay_sum as OS
    spec = synthetic_spec(n_rows=16 * 2000, seed=71)
    tab = G.device_table(spec, "q8_0", 16 * 2000, 128, seed=72)
    fetch = G.synth_fetch("q8_0", 72, 128)
    rng = np.random.default_rng(73)
    always = np.array([5, 7000, 31999])  # in every file
    paths, files = [], []
    for i in range(n_files):
        rows = np.unique(np.concatenate([rng.choice(16 * 2000, size=int(rng.integers(20, 60)), replace=False),
                                         always])).astype(np.int32)
        data = (fetch(rows) + rng.standard_normal((rows.size, 128)) * 1e-2).astype(np.float32)
        data[::4] = fetch(rows[::4])
        if i == 1:  # a row listed twice in one file: both deltas count, in file order
            rows = np.concatenate([rows, rows[-1:]])
            data = np.concatenate([data, data[-1:] + np.float32(1e-3)])
        path = tmp_path / f"f{i}.pleo"
        lens.write_pleo(path, rows, data)
        paths.append(path)
        files.append((rows, data))
    rows_u, merged, man = overlay_sum.sum_overlays(tab, paths)
    e_rows, e_merged, e_man = OS.sum_overlays(files, fetch)
    assert np.array_equal(rows_u, e_rows)
    assert np.array_equal(merged, e_merged)
    for k in ("n_files", "n_rows_union", "n_rows_moved_any", "n_rows_shared", "facts_per_row_histogram"):
        assert man[k] == e_man[k], k
    for k in ("shared_rows_sum_abs_norm_max", "shared_rows_abs_sum_norm_max", "max_row_delta_norm"):
        assert man[k] == pytest.approx(e_man[k], rel=1e-9), k
    r, d = overlay_sum.delta_for_pleo(tab, paths[0])
    assert np.array_equal(d, (files[0][1] - fetch(files[0][0])).astype(np.float32))
    # merged.pleo: variables in row_map order, then frozen rows ascending at true values
    row_map = {int(e_rows[3]): 0, int(e_rows[1]): 1}
    rv = torch.full((2, 128), 0.25)
    info = overlay_sum.write_merged_pleo(tab, row_map, rv, e_rows[:10].tolist(), tmp_path / "merged.pleo")
    got_rows, got_data = lens.read_pleo(tmp_path / "merged.pleo")
    exp_rows, exp_data = OS.write_merged_rows(row_map, rv.numpy(), e_rows[:10].tolist(), fetch)
    assert np.array_equal(got_rows, exp_rows) and np.array_equal(got_data, exp_data)
    assert info["n_rows_frozen"] == 8


def test_lookup_rows_sorted_search_edges(cuda):
    """eg_lookup_rows' search of the sorted ids (the same search resolves the
    forward's overlay ids) against numpy's searchsorted: every size from 1 to
    40 ids and 500,000, keys present, absent between ids, below the first and
    above the last; the read counts of the found ids."""
    from engraft_ngram_amd import _lib
    _say("sorted-id search edges")
    rng = np.random.default_rng(41)
    for n in list(range(1, 41)) + [500_000]:
        ids = np.unique(rng.integers(0, 2**31 - 2, size=2 * n))[:n].astype(np.int32)
        keys = np.concatenate([ids, ids - 1, ids + 1, [0, 2**31 - 1]]).astype(np.int32)
        if n > 40:
            keys = keys[rng.choice(keys.size, 20_000, replace=False)]
        pos = np.searchsorted(ids, keys)
        hit = (pos < n) & (ids[np.minimum(pos, n - 1)] == keys)
        exp = np.where(hit, pos, -1).astype(np.int32)
        ids_d = torch.from_numpy(ids).to(cuda)
        keys_d = torch.from_numpy(keys).to(cuda)
        out = torch.empty_like(keys_d)
        counts = torch.zeros(n, dtype=torch.int64, device=cuda)
        _lib.call("eg_lookup_rows", _lib.ptr(keys_d), keys.size, _lib.ptr(ids_d), None, n, _lib.ptr(out),
                  _lib.ptr(counts), _lib.stream_ptr(cuda))
        assert np.array_equal(out.cpu().numpy(), exp), n
        assert np.array_equal(counts.cpu().numpy(), np.bincount(exp[exp >= 0], minlength=n)), n


def test_exclusive_rows_at_position_against_oracle(cuda):
    """engraft/replica/seq.py:924-941 from one device hash: against the
    oracle's per-position RowSet loop on a stream whose n-grams repeat (rows
    reused at other positions), at the first, a middle and the last position,
    a position past n_positions, a negative position, and a head subset."""
    from engraft_ngram_amd import seq
    _say("exclusive_rows_at_position")
    spec = fake_table_spec(11, head_vocab_size=200)  # 6 token values: bigrams repeat, trigrams less
    tab, _ = G.f32_table(spec, 32, seed=12)
    rng = np.random.default_rng(13)
    tokens = rng.integers(0, 6, 60).tolist()
    tokens[20] = spec.eos_token_id
    n_pos = 48
    cases = [(0, None), (17, None), (n_pos - 1, None), (len(tokens) - 1, None), (-1, None), (-13, None),
             (30, range(0, 8)), (5, range(8, 16))]
    sizes = []
    for p, heads in cases:
        got = seq.exclusive_rows_at_position(tab, tokens, n_pos, p, heads)
        want = OE.exclusive_rows_at_position(spec, tokens, n_pos, p, heads)
        assert got == want, (p, heads)
        sizes.append(len(got))
    # whole sets, sets cut by rows reused elsewhere, and empty ones all occur
    assert 16 in sizes and 0 in sizes and any(0 < k < 16 for k in sizes[:6])
    # a row read again at another position is excluded: repeat position 3's window at 40
    tokens2 = list(tokens)
    tokens2[38:41] = tokens2[1:4]
    got = seq.exclusive_rows_at_position(tab, tokens2, 45, 3)
    assert got == OE.exclusive_rows_at_position(spec, tokens2, 45, 3) == set()
    with pytest.raises(IndexError):
        seq.exclusive_rows_at_position(tab, tokens, len(tokens) + 1, 0)
