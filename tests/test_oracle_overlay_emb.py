"""Pins of the OverlayEmb / ple_true_emb / damage-scan oracles (CPU)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import backward as B
from oracle import damage as DM
from oracle import forward as FW
from oracle import hash as H
from oracle import overlay_emb as OE
from oracle import synth
from tests.params import fake_table_spec, reference_corpus


def _fetch(spec, dim=32, seed=5):
    n = sum(spec.head_vocab_sizes)
    data = np.random.default_rng(seed).standard_normal((n, dim)).astype(np.float32) * 0.05
    return lambda ids: data[np.asarray(ids, dtype=np.int64)]


def test_build_replaces_mapped_rows_only():
    """tests/test_replica_graft.py:43-70 at sequence level: every slot whose
    global row is in row_map reads rows_var, every other slot is the plain
    gather bit for bit; an empty map is the plain gather."""
    spec = fake_table_spec(3, head_vocab_size=40)
    fetch = _fetch(spec)
    tokens = [int(x) for x in np.random.default_rng(1).integers(0, 6, 60)]
    rows = H.ngram_rows_np(spec, tokens)
    plain = FW.gather(rows, fetch)
    emb0, idx0, nk0, ni0 = OE.build(spec, tokens, {}, np.zeros((0, 32)), 60, fetch)
    assert np.array_equal(emb0, plain) and idx0 == ([], [], []) and nk0 == ni0 == 0
    picked = sorted(set(rows[::7, 3].tolist()) | set(rows[5::11, 12].tolist()))
    row_map = {g: i for i, g in enumerate(picked)}
    rv = np.random.default_rng(2).standard_normal((len(picked), 32)).astype(np.float32)
    emb, (it, ih, ir), nk, ni = OE.build(spec, tokens, row_map, rv, 60, fetch)
    e3, p3 = emb.reshape(60, 16, 32), plain.reshape(60, 16, 32)
    hit = np.isin(rows, picked)
    assert ni == int(hit.sum()) == len(it) and nk == 0
    for t in range(60):
        for h in range(16):
            exp = rv[row_map[int(rows[t, h])]] if hit[t, h] else p3[t, h]
            assert np.array_equal(e3[t, h], exp)


def test_long_key_wins_and_needs_full_window():
    spec = fake_table_spec(4, head_vocab_size=40)
    fetch = _fetch(spec)
    tokens = [1, 2, 3, 1, 2, 3, 9, 1, 2]
    rows = H.ngram_rows_np(spec, tokens)
    g = int(rows[2, 5])
    row_map = {g: 0, ((1, 2), 5): 1, ((2, 3), 5): 2}
    _, (it, ih, ir), nk, ni = OE.build(spec, tokens, row_map, np.zeros((3, 32), np.float32), 9, fetch)
    got = {(t, h): r for t, h, r in zip(it, ih, ir)}
    # windows (1,2) end at t=1,4,8 and (2,3) at t=2,5: key hits on head 5
    for t in (1, 4, 8):
        assert got[(t, 5)] == 1
    for t in (2, 5):
        assert got[(t, 5)] == 2
    assert nk == 5
    # an id hit elsewhere still counts as an id hit
    id_hits = {(t, h) for t in range(9) for h in range(16) if rows[t, h] == g and (t, h) not in
               {(1, 5), (4, 5), (8, 5), (2, 5), (5, 5)}}
    assert ni == len(id_hits)
    # position 0 cannot take a 2-token window even if its padded context would match
    assert (0, 5) not in got or got[(0, 5)] == 0


def test_segment_rule_equals_isolated_fragments():
    """engraft/replica/seq.py:263-271: with segment_ids every position hashes
    only its own segment -- equal to hashing each [EOS]+frag alone."""
    spec = fake_table_spec(5, head_vocab_size=40)
    fetch = _fetch(spec)
    eos = spec.eos_token_id
    frags = [[3, 5, 7, 2], [9, 4, 6], [4, 4, 4, 4, 4]]
    tokens, seg = [], []
    for i, f in enumerate(frags):
        tokens += [eos] + f
        seg += [i] * (len(f) + 1)
    n = len(tokens)
    rows_seg, *_ = OE.build_plan(spec, tokens, {}, n, 0, seg)
    iso = np.concatenate([H.ngram_rows_np(spec, [eos] + f) for f in frags])
    assert np.array_equal(rows_seg, iso)
    # ...and the vectorized hash with the segment starts agrees
    assert np.array_equal(H.ngram_rows_np(spec, tokens, seg_start=H.seg_starts_from_segment_ids(seg)), iso)


def test_gradient_equals_torch_index_put_autograd():
    """The gradient of rows_var through base.index_put((idx_t, idx_h),
    rows_var[idx_r]) by torch's own autograd on the CPU, against
    scatter_grad_keys over the slot map (bit-exact: every segment is short)."""
    spec = fake_table_spec(6, head_vocab_size=30)
    fetch = _fetch(spec)
    tokens = [int(x) for x in np.random.default_rng(3).integers(0, 5, 80)]
    rows = H.ngram_rows_np(spec, tokens)
    picked = sorted(set(rows[::3, 1].tolist()) | set(rows[::5, 9].tolist()))
    row_map = {g: i for i, g in enumerate(picked)}
    rv0 = np.random.default_rng(4).standard_normal((len(picked), 32)).astype(np.float32)
    _, base, it, ih, ir, _, _ = OE.build_plan(spec, tokens, row_map, 80, 0, None, fetch)
    rv = torch.from_numpy(rv0.copy()).requires_grad_(True)
    emb = torch.from_numpy(base).index_put((torch.tensor(it), torch.tensor(ih)), rv[torch.tensor(ir)])
    d = torch.from_numpy(np.random.default_rng(5).standard_normal((80, 16 * 32)).astype(np.float32))
    (emb.reshape(80, -1) * d).sum().backward()
    keys = OE.slot_keys(it, ih, ir, 80, 16)
    grad, hits = B.scatter_grad_keys(d.numpy(), keys, 16, len(picked))
    assert hits.max() <= B.PIECE
    assert np.array_equal(grad, rv.grad.numpy())


def test_ple_true_emb_matches_rowset_and_overlay():
    spec = fake_table_spec(7, head_vocab_size=50)
    fetch = _fetch(spec)
    tokens = [1, 2, 3, 4, 5]
    rows, data = OE.row_set(spec, tokens, 3, fetch)
    plain = OE.ple_true_emb(spec, tokens, 3, fetch)
    assert np.array_equal(plain, data.reshape(1, -1))
    vec = np.full(32, 99.0, np.float32)
    out = OE.ple_true_emb(spec, tokens, 3, fetch, {int(rows[0]): vec}).reshape(16, 32)
    assert np.array_equal(out[0], vec) and np.array_equal(out[1:], data[1:])


def _pick_rows(spec, tokens):
    rows = H.ngram_rows_np(spec, tokens)
    picks = [(100, 0), (150, 8 + 3), (300, 7), (777, 8 + 1), (5000, 5)]
    return np.array(sorted({int(rows[p, h]) for p, h in picks}), dtype=np.int64)


def test_scan_hits_reference_known_answer():
    """tests/test_damage.py:38-61: seed-7 FakeTable parameters, 20,000 tokens,
    EOS every 200, block 4,000; hits on the first 2,000 positions equal the
    scalar ngram_addresses loop; the last position is never a hit."""
    spec = fake_table_spec(7)
    tokens = reference_corpus(20_000, seed=1, eos=spec.eos_token_id)
    ov = _pick_rows(spec, tokens)
    dn = np.arange(1, ov.size + 1, dtype=np.float32)
    hits = DM.scan_hits(spec, tokens, ov, dn, block=4_000)
    addr = H.ngram_addresses_scalar(spec, tokens[:2000].tolist())
    ovs = set(ov.tolist())
    exp = {p for p in range(1999) if ovs & {H.local_to_global(spec, h, addr[p][h]) for h in range(16)}}
    assert {int(p) for p in hits["pos"] if p < 2000} == exp
    assert 19_999 not in set(hits["pos"].tolist())
    # block-size independent, read_count = brute-force count over all positions
    one = DM.scan_hits(spec, tokens, ov, dn, block=20_000)
    for k in ("pos", "n_hit_rows", "dnorm_max", "dnorm_sum", "read_count"):
        assert np.array_equal(hits[k], one[k])
    rows = H.ngram_rows_np(spec, tokens)
    assert hits["read_count"].tolist() == [int((rows == g).sum()) for g in ov]


def _files(rng, fetch, n_files, pool, dim=32, unchanged_every=3):
    files = []
    for i in range(n_files):
        rows = np.sort(rng.choice(pool, size=min(pool, int(rng.integers(5, 12))), replace=False)).astype(np.int32)
        data = fetch(rows) + rng.standard_normal((rows.size, dim)).astype(np.float32) * 1e-2
        data[::unchanged_every] = fetch(rows[::unchanged_every])  # rows the fact left untouched
        files.append((rows, data.astype(np.float32)))
    return files


@pytest.mark.parametrize("n_files,pool", [(5, 40), (40, 6)])
def test_overlay_sum_against_dict_loop(n_files, pool):
    """engraft/replica/overlay_sum.py:38-112 by a per-row dictionary loop:
    union ascending, deltas added one at a time in file order (40 files put
    far more than 32 deltas on the rows of a 40-row pool; one file lists a
    row twice), merged = true + sum; an untouched row's delta is exactly zero
    and is not counted as moved."""
    from oracle import overlay_sum as OS
    data = np.random.default_rng(8).standard_normal((500, 32)).astype(np.float32) * 0.05
    fetch = lambda ids: data[np.asarray(ids, np.int64)]
    rng = np.random.default_rng(9)
    files = _files(rng, fetch, n_files, pool)
    r0, d0 = files[1]
    files[1] = (np.concatenate([r0, r0[:1]]), np.concatenate([d0, d0[:1] + np.float32(3e-3)]))
    rows_u, merged, man = OS.sum_overlays(files, fetch)
    acc: dict[int, np.ndarray] = {}
    moved: dict[int, int] = {}
    for rows, d in files:
        for r, v in zip(rows.tolist(), d):
            delta = (v - data[r]).astype(np.float32)
            acc[r] = (acc.get(r, np.zeros(32, np.float32)) + delta).astype(np.float32)
            if np.linalg.norm(delta.astype(np.float64)) > 0:
                moved[r] = moved.get(r, 0) + 1
    assert rows_u.tolist() == sorted(acc)
    hits = np.bincount(np.concatenate([r for r, _ in files]))
    assert (hits.max() > 32) == (n_files == 40)
    for i, r in enumerate(rows_u.tolist()):
        assert np.array_equal(merged[i], (data[r] + acc[r]).astype(np.float32))
    assert man["n_rows_moved_any"] == len(moved)
    assert man["n_rows_shared"] == sum(1 for c in moved.values() if c >= 2)
    assert sum(man["facts_per_row_histogram"].values()) == len(moved)
    # one file alone: merged == true + (data - true), untouched rows bit-identical
    r1, m1, man1 = OS.sum_overlays(files[:1], fetch)
    assert np.array_equal(m1[::3], files[0][1][::3]) and man1["n_rows_shared"] == 0


def test_write_merged_rows_order():
    """engraft/descend_corpus.py:627-647: variables in row_map order, then the
    frozen rows ascending at their true values (not globally sorted)."""
    from oracle import overlay_sum as OS
    data = np.arange(50 * 4, dtype=np.float32).reshape(50, 4)
    fetch = lambda ids: data[np.asarray(ids, np.int64)]
    row_map = {30: 0, 7: 1}
    rv = np.full((2, 4), -1.0, np.float32)
    rows, d = OS.write_merged_rows(row_map, rv, [3, 30, 12, 7, 3], fetch)
    assert rows.tolist() == [30, 7, 3, 12]
    assert np.array_equal(d[:2], rv) and np.array_equal(d[2:], data[[3, 12]])


def test_exclusive_rows_known_answers():
    """``engraft/replica/seq.py:924-941`` on streams built so the answer is fixed
    by the window rule alone (position t's order-n rows depend only on tokens
    t-n+1..t): a window repeated at another position inside ``n_positions``
    empties the set, the same repeat past ``n_positions`` leaves all 16 rows,
    a shared 2-gram with different 3-grams leaves exactly the order-3 heads'
    rows (heads 8..15), and ``p`` itself is never subtracted.  Large head
    vocabularies keep hash collisions between the few distinct windows out."""
    spec = fake_table_spec(2, head_vocab_size=1_000_003)
    a, b, c, x, y = 11, 12, 13, 14, 15
    toks = [a, b, c, x, a, b, c]
    rows = H.ngram_rows_np(spec, toks)
    assert np.array_equal(rows[2], rows[6])  # the construction: same window
    assert OE.exclusive_rows_at_position(spec, toks, 7, 2) == set()
    assert OE.exclusive_rows_at_position(spec, toks, 7, 6) == set()
    assert OE.exclusive_rows_at_position(spec, toks, 6, 2) == {int(r) for r in rows[2]}
    assert OE.exclusive_rows_at_position(spec, toks, 7, 3) == {int(r) for r in rows[3]}
    toks2 = [a, b, c, y, b, c]
    rows2 = H.ngram_rows_np(spec, toks2)
    got = OE.exclusive_rows_at_position(spec, toks2, 6, 2)
    assert got == {int(r) for r in rows2[2, 8:]} and len(got) == 8
    assert OE.exclusive_rows_at_position(spec, toks2, 6, 2, heads=range(0, 8)) == set()
    assert OE.exclusive_rows_at_position(spec, toks2, 6, 2, heads=range(8, 10)) == {int(r) for r in rows2[2, 8:10]}
