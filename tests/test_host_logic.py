"""Host-side logic of the drop-in (no GPU): packing, ``.pleo`` IO,
``build_overlay``, ``overlay_key_len``, block iteration -- against the
reference's own tests and fixtures."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import hash as H

GOLDEN = Path(__file__).parent / "golden"


def _pkg():
    from engraft_ngram_amd import damage, lens, pack, seq  # noqa: F401
    return lens, pack, seq, damage


def test_pack_segment_ids_reference_case():
    """tests/test_seq.py:54-57: frags [3,5,7,2], [9,4,6] -> one bin, segment
    ids [0,0,0,0,0,1,1,1]."""
    _, pack, _, _ = _pkg()
    p = pack.pack_fragments([[3, 5, 7, 2], [9, 4, 6]], 99, max_len=64)
    assert len(p) == 1
    p = p[0]
    assert p.tokens == [99, 3, 5, 7, 2, 99, 9, 4, 6]
    assert p.segment_ids.tolist() == [0, 0, 0, 0, 0, 1, 1, 1]
    assert p.positions.tolist() == [0, 1, 2, 3, 4, 0, 1, 2]
    assert p.frag_slices == [(0, 4), (5, 8)]
    assert p.seg_start().tolist() == [0, 0, 0, 0, 0, 5, 5, 5]
    assert p.seg_start().tolist() == H.seg_starts_from_segment_ids(p.segment_ids.numpy()).tolist()


def test_pack_greedy_bins_and_oversize():
    _, pack, _, _ = _pkg()
    frags = [[1] * 5, [2] * 5, [3] * 3, [4] * 9]
    bins = pack.pack_fragments(frags, 0, max_len=10)
    # canonical lengths 6, 6, 4, 10 -> [6], [6, 4], [10]
    assert [len(b.tokens) for b in bins] == [6, 10, 10]
    assert bins[1].segment_ids.tolist() == [0] * 6 + [1] * 3
    with pytest.raises(ValueError):
        pack.pack_fragments([[1] * 10], 0, max_len=10)
    assert pack.pack_fragments([], 0, max_len=10) == []


@pytest.mark.parametrize("seed", range(6))
def test_pack_invariants_random(seed):
    """Invariants that fix greedy in-order packing whatever the implementation:
    the bins concatenate to ``[eos]+frag`` for every fragment in order; no bin
    exceeds ``max_len``; the next bin's first fragment would not have fitted;
    every prefix position's segment id and offset point back at its
    fragment's leading EOS; each frag slice spans the fragment's ``len(frag)``
    significant positions."""
    _, pack, _, _ = _pkg()
    rng = np.random.default_rng(seed)
    max_len = int(rng.integers(4, 40))
    frags = [rng.integers(1, 50, size=int(rng.integers(0, max_len))).tolist()
             for _ in range(int(rng.integers(0, 30)))]
    eos = 0
    bins = pack.pack_fragments(frags, eos, max_len)
    flat = [t for b in bins for t in b.tokens]
    assert flat == [t for f in frags for t in [eos] + f]
    k = 0  # fragments consumed so far
    for i, b in enumerate(bins):
        assert len(b.tokens) <= max_len
        n_frag = len(b.frag_slices)
        assert n_frag >= 1
        if i + 1 < len(bins):
            assert len(b.tokens) + len(frags[k + n_frag]) + 1 > max_len
        n_prefix = len(b.tokens) - 1
        seg = b.segment_ids.numpy()
        pos = b.positions.numpy()
        assert seg.shape == (n_prefix,) and pos.shape == (n_prefix,)
        for j in range(n_prefix):
            start = j - int(pos[j])
            assert b.tokens[start] == eos
            assert b.frag_slices[int(seg[j])][0] == start
        for s_i, (a, e) in enumerate(b.frag_slices):
            assert e - a == len(frags[k + s_i])
            assert b.tokens[a] == eos
        k += n_frag
    assert k == len(frags)


@pytest.mark.parametrize("seed", range(4))
def test_build_overlay_matches_first_wins_dedup(seed):
    """build_overlay against the plain specification: every row once,
    ascending, with the vector it was given (all copies equal)."""
    lens, _, _, _ = _pkg()
    rng = np.random.default_rng(seed)
    truth = {int(r): rng.standard_normal(8).astype(np.float32) for r in rng.choice(1000, 40, replace=False)}
    keys = list(truth)
    parts = []
    for _ in range(int(rng.integers(1, 5))):
        pick = rng.choice(keys, int(rng.integers(0, 30)))
        parts.append((np.array(pick, dtype=np.int64), np.stack([truth[int(r)] for r in pick])
                      if len(pick) else np.zeros((0, 8), np.float32)))
    rows, data = lens.RowSet.build_overlay(parts)
    want = sorted({int(x) for r, _ in parts for x in r})
    assert rows.tolist() == want and rows.dtype == np.int32
    for r, v in zip(rows.tolist(), data):
        np.testing.assert_array_equal(v, truth[r])
    if want:
        bad = np.stack([truth[want[0]] + 1.0])
        with pytest.raises(ValueError):
            lens.RowSet.build_overlay(parts + [(np.array([want[0]]), bad)])


def test_pleo_roundtrip_and_bad_magic(tmp_path):
    """tests/test_lens.py:57-72."""
    lens, _, _, _ = _pkg()
    rows = np.array([5, 100000, 3, 999999999], dtype=np.int32)
    data = np.random.default_rng(0).standard_normal((4, 160)).astype(np.float32)
    path = tmp_path / "x.pleo"
    lens.write_pleo(path, rows, data)
    r, d = lens.read_pleo(path)
    np.testing.assert_array_equal(r, rows)
    np.testing.assert_array_equal(d, data)
    bad = tmp_path / "bad.pleo"
    bad.write_bytes(b"NOPE" + b"\x00" * 20)
    with pytest.raises(ValueError):
        lens.read_pleo(bad)
    with pytest.raises(ValueError):
        lens.write_pleo(path, rows, data[:3])


@pytest.mark.parametrize("name,n_rows", [("real_en_dog.pleo", 16), ("real_it_gatto.pleo", 48)])
def test_pleo_real_fixtures_byte_exact(tmp_path, name, n_rows):
    """Real overlays written by the reference (results/2026-09-05/facts/*):
    read, then written back byte for byte."""
    lens, _, _, _ = _pkg()
    src = GOLDEN / name
    rows, data = lens.read_pleo(src)
    assert rows.shape == (n_rows,) and data.shape == (n_rows, 160)
    assert np.all(np.isfinite(data))
    assert 0 < float(np.abs(data).max()) < 1.0
    out = tmp_path / name
    lens.write_pleo(out, rows, data)
    assert out.read_bytes() == src.read_bytes()


def test_build_overlay_dedup_and_conflict():
    """tests/test_lens.py:184-208."""
    lens, _, _, _ = _pkg()
    rows1 = np.array([5, 10], dtype=np.int32)
    data1 = np.ones((2, 160), dtype=np.float32)
    rows2 = np.array([10, 20], dtype=np.int32)
    data2 = np.stack([np.ones(160, np.float32), np.full(160, 2.0, np.float32)])
    rows, data = lens.RowSet.build_overlay([(rows1, data1), (rows2, data2)])
    assert rows.tolist() == [5, 10, 20]
    np.testing.assert_array_equal(data[2], np.full(160, 2.0))
    with pytest.raises(ValueError):
        lens.RowSet.build_overlay([(np.array([5]), np.ones((1, 160), np.float32)),
                                   (np.array([5]), np.full((1, 160), 2.0, np.float32))])


def _build_overlay_dict_loop(parts):
    """The reference's dict loop (``engraft/lens.py:177-198``) as a plain
    specification: a row's first vector is stored without any comparison,
    every later one must be ``np.array_equal`` to it."""
    seen = {}
    for rows_global, data in parts:
        for r, vec in zip(np.asarray(rows_global).tolist(), np.asarray(data, np.float32)):
            if r in seen:
                if not np.array_equal(seen[r], vec):
                    raise ValueError(r)
            else:
                seen[r] = vec
    keys = sorted(seen)
    return np.array(keys, np.int32), np.stack([seen[k] for k in keys])


def test_build_overlay_nan_row_seen_once_is_accepted():
    """A NaN-bearing row listed once is stored as given, NaN bits and all;
    a row with a NaN listed twice is rejected, as np.array_equal rejects it."""
    lens, _, _, _ = _pkg()
    d = np.arange(2 * 6, dtype=np.float32).reshape(2, 6)
    d[1, 3] = np.nan
    parts = [(np.array([5, 9]), d), (np.array([5]), d[:1].copy())]
    rows, data = lens.RowSet.build_overlay(parts)
    want_rows, want_data = _build_overlay_dict_loop(parts)
    assert rows.tolist() == want_rows.tolist() == [5, 9]
    assert data.tobytes() == want_data.tobytes()
    assert np.isnan(data[1, 3]) and np.isfinite(np.delete(data[1], 3)).all()
    twice = [(np.array([9]), d[1:]), (np.array([9]), d[1:].copy())]
    with pytest.raises(ValueError):
        _build_overlay_dict_loop(twice)
    with pytest.raises(ValueError):
        lens.RowSet.build_overlay(twice)


def test_build_overlay_signed_zero_equal():
    """-0.0 and 0.0 compare equal under np.array_equal, so a row carrying
    both is accepted, and the first member's bits are kept."""
    lens, _, _, _ = _pkg()
    a = np.zeros((1, 4), np.float32)
    b = a.copy()
    b[0, 2] = -0.0
    rows, data = lens.RowSet.build_overlay([(np.array([3]), b), (np.array([3]), a)])
    want_rows, want_data = _build_overlay_dict_loop([(np.array([3]), b), (np.array([3]), a)])
    assert rows.tolist() == want_rows.tolist() == [3]
    assert data.tobytes() == want_data.tobytes() == b.tobytes()


def test_overlay_key_len():
    _, _, seq, _ = _pkg()
    assert seq.overlay_key_len({1: 0, 7: 1}) is None
    assert seq.overlay_key_len({1: 0, ((3, 4, 5), 2): 1}) == 3
    with pytest.raises(AssertionError):
        seq.overlay_key_len({((3, 4), 2): 0, ((3, 4, 5), 2): 1})


def test_iter_blocks_overlap():
    """engraft/damage.py:107-118: 2 tokens of history except on the first block."""
    _, _, _, damage = _pkg()
    toks = np.arange(10)
    blocks = list(damage.iter_blocks(toks, block=4))
    assert [o for o, _ in blocks] == [0, 4, 8]
    assert [b.tolist() for _, b in blocks] == [[0, 1, 2, 3], [2, 3, 4, 5, 6, 7], [6, 7, 8, 9]]


def test_gguf_reader_layout(tmp_path):
    """The GGUF directory as the published format lays it out: typed metadata
    (scalars, strings, arrays), tensor dims ne0-first, data offsets aligned to
    general.alignment and pointing at each tensor's bytes."""
    from engraft_ngram_amd.ggufio import read_gguf
    from tests.gguf_util import ple_table_file
    from tests.params import fake_table_spec

    spec = fake_table_spec(3, head_vocab_size=7)
    rng = np.random.default_rng(0)
    raw = [rng.integers(0, 256, size=(7, 90), dtype=np.uint8) for _ in range(16)]
    offs = ple_table_file(tmp_path / "t.gguf", spec, raw)
    g = read_gguf(tmp_path / "t.gguf")
    assert g.version == 3 and g.alignment == 32
    assert g.fields["general.architecture"] == "qwen4exp"
    assert g.fields["qwen4exp.ple.layer_multipliers"] == list(spec.layer_multipliers)
    assert g.fields["qwen4exp.ple.head_offsets"] == list(spec.head_offsets)
    data = (tmp_path / "t.gguf").read_bytes()
    for h in range(16):
        t = g.tensors[f"ple_ngram_embd.{h}.weight"]
        assert t.shape == (160, 7) and t.ggml_type == 20 and t.data_offset == offs[h]
        assert t.data_offset % 32 == 0
        assert data[t.data_offset:t.data_offset + 630] == raw[h].tobytes()
    (tmp_path / "bad.gguf").write_bytes(b"GGML" + b"\0" * 40)
    with pytest.raises(ValueError):
        read_gguf(tmp_path / "bad.gguf")


def _ple_w(hc=4, n=64, taps=4, seed=0):
    rng = np.random.default_rng(seed)
    f = lambda *s, sc=1.0: (rng.standard_normal(s) * sc).astype(np.float32)
    return {"w_key": f(hc * n, n, sc=n ** -0.5), "w_value": f(n, n, sc=n ** -0.5), "norm_key": 1 + f(hc * n, sc=0.1),
            "norm_query": 1 + f(hc * n, sc=0.1), "norm_conv": 1 + f(hc * n, sc=0.1), "conv1d": f(hc * n, taps)}


def test_gguf_ple_weights_reader(tmp_path):
    """The PLE weights of a model GGUF (engraft/lens.py:229-266): Q8_0 and F32
    tensors read to their closed-form values (d*q), the type check, and the
    RMS epsilon from shard 1 of a split (lens.py:490-518)."""
    from engraft_ngram_amd import ggufio
    from tests import gguf_util as GU
    w = _ple_w()
    path, vals = GU.ple_model_files(tmp_path, w, 1e-6)
    gf = ggufio.read_gguf(path)
    for name, ref in vals.items():
        got = ggufio.read_tensor_f32(gf, f"blk.1.ple_{name.replace('w_', '')}.weight")
        assert got.shape == np.asarray(ref).shape
        assert np.array_equal(got, ref)
    # Q8_0 values are within half a step of the source
    assert np.abs(vals["w_value"] - w["w_value"]).max() <= np.abs(w["w_value"]).max() / 127
    with pytest.raises(ValueError):
        ggufio.read_tensor_f32(gf, "blk.1.ple_key.weight", expected_type=ggufio.GGML_TYPE_F32)
    with pytest.raises(KeyError):
        ggufio.read_tensor_f32(gf, "blk.2.ple_key.weight")
    assert ggufio.read_rms_eps(path) == np.float32(1e-6)
    (tmp_path / "one").mkdir()
    one, _ = GU.ple_model_files(tmp_path / "one", w, 1e-5, split=False)
    assert ggufio.read_rms_eps(one) == np.float32(1e-5)
    (tmp_path / "m-00001-of-00002.gguf").unlink()
    with pytest.raises(FileNotFoundError):
        ggufio.read_rms_eps(path)
    GU.write_gguf(tmp_path / "m-00001-of-00002.gguf", [("general.architecture", GU.STRING, "qwen4exp")], [])
    with pytest.raises(KeyError):
        ggufio.read_rms_eps(path)


def test_rowstore_padded_iq4nl_rows():
    """IQ4_NL rows in 128-byte lines: the payload's wider rows are accepted
    (even strides only), the C table carries the stride, raw rows drop the
    padding, and no other format takes a stride."""
    import torch

    from engraft_ngram_amd import table as T
    assert T.RowStore.padded_stride("iq4_nl", 160) == 128
    assert T.RowStore.padded_stride("iq4_nl", 256) == 256  # 144 bytes -> two lines
    assert T.RowStore.padded_stride("q8_0", 128) == 128
    st = T.RowStore.empty("iq4_nl", 6, 160, "cpu", row_stride=128)
    assert tuple(st.payload.shape) == (6, 128) and st.row_bytes == 90 and st.row_stride == 128
    assert st.c_table().row_stride == 128
    rng = np.random.default_rng(5)
    st.payload.copy_(torch.from_numpy(rng.integers(0, 256, size=(6, 128), dtype=np.uint8)))
    got = st.raw_rows(torch.tensor([4, 1]))
    assert got.shape == (2, 90) and np.array_equal(got, st.payload.numpy()[[4, 1], :90])
    plain = T.RowStore.empty("iq4_nl", 6, 160, "cpu")
    assert plain.row_stride == 0 and plain.c_table().row_stride == 0 and plain.row_bytes == 90
    with pytest.raises(ValueError):
        T.RowStore("iq4_nl", 160, torch.zeros((6, 127), dtype=torch.uint8))
    with pytest.raises(ValueError):
        T.RowStore("iq4_nl", 160, torch.zeros((6, 88), dtype=torch.uint8))
    with pytest.raises(ValueError):
        T.RowStore.empty("q8_0", 6, 128, "cpu", row_stride=256)
