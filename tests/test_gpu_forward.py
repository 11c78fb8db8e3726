"""GPU parity of the forward path (hash, synthetic rows, gather, fused
hash -> gather -> dequant -> overlay -> residual add) against the CPU oracle.

Bar: row ids bit-exact; dequantised rows bit-exact; outputs within 1e-3
relative of the oracle (bf16 out, fp32 accumulate) -- and, since every step is
exact or IEEE-rounded once, bit-exact in practice, which is asserted too."""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import forward as FW
from oracle import hash as H
from oracle import synth
from tests import gpu_util as G
from tests.params import CFG0, CFG1, CFG3, CFG4, fake_table_spec, reference_corpus, synthetic_spec, tiny_hparams_spec

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


@pytest.mark.parametrize("fmt", ["q8_0", "bf16", "mxfp8"])
def test_synthetic_rows_match_oracle_bytes(cuda, fmt):
    _say(f"synth {fmt}")
    n, dim, seed = 5000, 128, 17
    spec = synthetic_spec(n_rows=16 * 300, seed=1)
    tab = G.device_table(spec, fmt, n, dim, seed)
    payload, scales = synth.synth_rows(fmt, seed, np.arange(n), dim, 0.02)
    got_p = tab.store.payload.view(torch.uint8).cpu().numpy().reshape(n, -1)
    assert np.array_equal(got_p, np.ascontiguousarray(payload).view(np.uint8).reshape(n, -1))
    if scales is not None:
        got_s = tab.store.scales.view(torch.uint8).cpu().numpy().reshape(n, -1)
        assert np.array_equal(got_s, np.ascontiguousarray(scales).view(np.uint8).reshape(n, -1))


@pytest.mark.parametrize("name,spec_fn", [
    ("fake7", lambda: fake_table_spec(7)),
    ("tiny", tiny_hparams_spec),
    ("synthetic", lambda: synthetic_spec(n_rows=16 * 262_144, seed=5)),
    ("4gram", lambda: synthetic_spec(n_rows=24 * 1000, seed=9, ngram_size=4)),
])
def test_hash_rows_match_oracle(cuda, name, spec_fn):
    """Reference corpus of tests/test_damage.py:19-23 (EOS every 200)."""
    _say(f"hash {name}")
    spec = spec_fn()
    n_rows = spec.head_offsets[-1] + spec.head_vocab_sizes[-1]
    tab = G.device_table(spec, "q8_0", n_rows, 128, seed=1)
    tokens = reference_corpus(eos=spec.eos_token_id)
    got = tab.rows(torch.from_numpy(tokens.astype(np.int64))).cpu().numpy()
    assert np.array_equal(got, H.ngram_rows_np(spec, tokens))
    got_local = tab.rows(torch.from_numpy(tokens.astype(np.int64)), global_ids=False).cpu().numpy()
    assert np.array_equal(got_local, H.ngram_rows_np(spec, tokens, global_ids=False))
    # the list-of-lists API of engraft/table.py:111-144 on a short prefix
    assert tab.ngram_addresses(tokens[:300].tolist()) == H.ngram_addresses_scalar(spec, tokens[:300].tolist())


def test_hash_unsigned_modulus_edges(cuda):
    """mixed = token (multipliers [1, 0]) walks uint64 edge values on the device."""
    p = 4999
    spec = H.HashSpec(eos_token_id=7, ngram_size=2, heads_per_ngram=3, layer_multipliers=(1, 0),
                      head_vocab_sizes=(p, 65521, 1_000_003), head_offsets=(0, p, p + 65521))
    tab = G.device_table(spec, "bf16", spec.head_offsets[-1] + spec.head_vocab_sizes[-1], 32, seed=0)
    vals = [0, 1, p - 1, p, 7 * p, 7 * p - 1, 2**32 - 1, 2**32, 2**63 - 1, 2**63, 2**63 + 1, 2**64 - 1,
            (2**64 - 1) - ((2**64 - 1) % p), 0xDEADBEEFCAFEBABE, 3 * 1_000_003 - 1]
    tokens = np.array([v - 2**64 if v >= 2**63 else v for v in vals], dtype=np.int64)
    got = tab.rows(torch.from_numpy(tokens), global_ids=False).cpu().numpy()
    exp = [[v % q for q in spec.head_vocab_sizes] for v in vals]
    assert got.tolist() == exp


def test_hash_segments_and_batch_rows(cuda):
    spec = fake_table_spec(1)
    tab = G.device_table(spec, "q8_0", 16 * 5000, 128, seed=2)
    tokens = np.array([spec.eos_token_id, 3, 5, 7, 2, spec.eos_token_id, 9, 4, 6], dtype=np.int64)
    seg_start = H.seg_starts_from_segment_ids([0, 0, 0, 0, 0, 1, 1, 1, 1])
    got = tab.rows(torch.from_numpy(tokens), seg_start=seg_start).cpu().numpy()
    assert np.array_equal(got, H.ngram_rows_np(spec, tokens, seg_start=seg_start))
    rng = np.random.default_rng(0)
    toks = rng.integers(0, 40, size=8 * 257)
    got = tab.rows(torch.from_numpy(toks), seq_len=257).cpu().numpy()
    assert np.array_equal(got, H.ngram_rows_np(spec, toks, seq_len=257))


def test_forward_config0_full_size(cuda):
    """BASELINE config 0 at its own size: 4,194,304-row bf16 table, 2048
    uniform tokens over 151,936 ids, residual [2048, 2048] bf16 ~ N(0, 1)."""
    _say("forward cfg0")
    c = CFG0
    spec = synthetic_spec(n_rows=c["n_rows"], seed=100)
    tab = G.device_table(spec, "bf16", c["n_rows"], c["dim"], seed=101)
    tokens = synth.uniform_tokens(102, c["seq"], c["vocab"])
    res = G.residual(c["seq"], c["width"], seed=103)
    out, rows = tab.forward(torch.from_numpy(tokens), res, return_rows=True)
    exp_rows, _, exp_out = FW.forward(spec, tokens, G.synth_fetch("bf16", 101, 128), G.bf16_bits(res))
    assert np.array_equal(rows[0].cpu().numpy(), exp_rows)
    G.assert_out_matches(G.bf16_bits(out), exp_out)


@pytest.mark.parametrize("fmt", ["q8_0", "mxfp8", "bf16"])
def test_forward_small_formats_and_emb_mode(cuda, fmt):
    spec = synthetic_spec(n_rows=16 * 4096, seed=7)
    n_rows = 16 * 4096
    tab = G.device_table(spec, fmt, n_rows, 128, seed=8)
    rng = np.random.default_rng(9)
    tokens = rng.integers(0, 3000, size=4 * 300)
    tokens[::41] = spec.eos_token_id
    fetch = G.synth_fetch(fmt, 8, 128)
    res = G.residual(tokens.size, 2048, seed=10)
    out = tab.forward(torch.from_numpy(tokens), res, seq_len=300)
    exp_rows, exp_emb, exp_out = FW.forward(spec, tokens, fetch, G.bf16_bits(res), seq_len=300)
    G.assert_out_matches(G.bf16_bits(out), exp_out)
    emb = tab.forward(torch.from_numpy(tokens), None, seq_len=300)
    assert emb.dtype == torch.float32
    assert np.array_equal(emb.cpu().numpy(), exp_emb)
    # in-place residual update (out aliases residual)
    res2 = res.clone()
    tab.forward(torch.from_numpy(tokens), res2, out=res2, seq_len=300)
    assert np.array_equal(G.bf16_bits(res2), exp_out)


def test_gather_read_rows_and_bounds(cuda):
    spec = synthetic_spec(n_rows=16 * 1000, seed=3)
    tab = G.device_table(spec, "q8_0", 16 * 1000, 128, seed=4)
    ids = np.array([[0, 5], [15999, 7], [123, 123]], dtype=np.int32)
    got = tab.gather(torch.from_numpy(ids)).cpu().numpy()
    exp = FW.gather(ids, G.synth_fetch("q8_0", 4, 128))
    assert np.array_equal(got, exp)
    # read_rows / read_rows_raw of engraft/table.py:90-109
    r = tab.read_rows(3, 10, 4)
    assert np.array_equal(r, G.synth_fetch("q8_0", 4, 128)(np.arange(3010, 3014)))
    raw = tab.read_rows_raw(3, 10, 4)
    assert raw.shape == (4, 4 * 34)
    with pytest.raises(AssertionError):
        tab.read_rows(3, 999, 2)
    # ids outside the table read NaN on the device, never memory
    bad = tab.gather(torch.tensor([[-1, 16000, 2**31 - 1]], dtype=torch.int32)).cpu().numpy()
    assert np.isnan(bad).all()


def test_iq4nl_real_format_gather(cuda):
    """The reference's real 90-byte IQ4_NL rows (engraft/table.py:147-169)."""
    from engraft_ngram_amd import table as T
    rng = np.random.default_rng(11)
    raw = rng.integers(0, 256, size=(777, 90), dtype=np.uint8)
    for b in range(5):  # finite fp16 scales
        raw[:, b * 18:b * 18 + 2] = (rng.standard_normal((777, 1)) * 0.01).astype(np.float16).view(np.uint8)
    got = T.dequant_iq4nl(raw)
    assert np.array_equal(got, G.F.dequant_iq4nl(raw))
    zero = np.zeros((4, 90), dtype=np.uint8)
    zero[1, 0] = 1
    zero[3, 19] = 0x80
    assert T.row_is_zero(zero).tolist() == [True, False, True, False]


def test_forward_overlay_f32_and_q8(cuda):
    """engraft/replica/model.py:473-495: overlay rows replace present ids, every
    other slot stays bit-identical (tests/test_replica_graft.py:43-70)."""
    from engraft_ngram_amd.overlay import DeviceOverlay
    spec = synthetic_spec(n_rows=16 * 2000, seed=21)
    tab = G.device_table(spec, "q8_0", 16 * 2000, 128, seed=22)
    rng = np.random.default_rng(23)
    tokens = rng.integers(0, 50, size=1024)
    fetch = G.synth_fetch("q8_0", 22, 128)
    rows = H.ngram_rows_np(spec, tokens)
    ov_ids = np.unique(rng.choice(np.unique(rows), size=300, replace=False)).astype(np.int32)
    ov_rows = (rng.standard_normal((ov_ids.size, 128)) * 0.05).astype(np.float32)
    res = G.residual(tokens.size, 2048, seed=24)
    for kind in ("f32", "q8_0"):
        if kind == "f32":
            ov = DeviceOverlay.from_rows(ov_ids, ov_rows, device=cuda)
            ov_vals = ov_rows
        else:
            q, d = G.F.quant_q8_0(ov_rows)
            ov = DeviceOverlay.from_quantized("q8_0", ov_ids, q, d, device=cuda)
            ov_vals = G.F.dequant_q8_0(q, d)
        out = tab.forward(torch.from_numpy(tokens), res, overlay=ov)
        _, _, exp_out = FW.forward(spec, tokens, fetch, G.bf16_bits(res), overlay=(ov_ids, ov_vals))
        G.assert_out_matches(G.bf16_bits(out), exp_out)
        emb = tab.gather(torch.from_numpy(rows.astype(np.int32)), overlay=ov).cpu().numpy()
        exp_emb, hits = FW.substitute(FW.gather(rows, fetch), rows, ov_ids, ov_vals)
        assert hits > 0 and np.array_equal(emb, exp_emb)


def test_forward_two_layer_mxfp8_4gram(cuda):
    """BASELINE config 4 shape at reduced rows: 2 layers x 24 heads (2-, 3-, 4-grams)
    of MXFP8 rows, residual width 3072, out = bf16(res + emb_0 + emb_1)."""
    from engraft_ngram_amd import table as T
    specs = [synthetic_spec(n_rows=24 * 5000, seed=31 + l, ngram_size=4) for l in range(2)]
    tabs = [G.device_table(specs[l], "mxfp8", 24 * 5000, 128, seed=41 + l) for l in range(2)]
    tokens = synth.zipf_tokens(50, 4096, 129_280)
    res = G.residual(4096, 3072, seed=51)
    out, rows = T.forward(tabs, torch.from_numpy(tokens), res, return_rows=True)
    embs = []
    for l in range(2):
        r, e, _ = FW.forward(specs[l], tokens, G.synth_fetch("mxfp8", 41 + l, 128))
        assert np.array_equal(rows[l].cpu().numpy(), r)
        embs.append(e)
    G.assert_out_matches(G.bf16_bits(out), FW.residual_add(G.bf16_bits(res), embs))


def test_forward_rows_equals_hashed_forward(cuda):
    """eg_forward_rows (ids given) against the oracle and against eg_forward on
    the same ids: one Q8_0 layer (the config-1 shape), one layer with an f32
    overlay, two MXFP8 4-gram layers (width 3072); an id outside the table reads
    NaN in its head's columns only."""
    from engraft_ngram_amd import table as T
    from engraft_ngram_amd.overlay import DeviceOverlay
    _say("forward_rows")
    spec = synthetic_spec(n_rows=16 * 3000, seed=121)
    tab = G.device_table(spec, "q8_0", 16 * 3000, 128, seed=122)
    tokens = synth.zipf_tokens(123, 2048, 5000)
    res = G.residual(2048, 2048, seed=124)
    out, rows = T.forward([tab], torch.from_numpy(tokens), res, return_rows=True)
    got = T.forward_rows([tab], rows, res)
    _, _, exp = FW.forward(spec, tokens, G.synth_fetch("q8_0", 122, 128), G.bf16_bits(res))
    G.assert_out_matches(G.bf16_bits(got), exp)
    assert torch.equal(got.view(torch.int16), out.view(torch.int16))
    # overlay resolved per id, as in eg_forward
    rng = np.random.default_rng(125)
    r_np = rows[0].cpu().numpy()
    ov_ids = np.unique(rng.choice(np.unique(r_np), size=200, replace=False)).astype(np.int32)
    ov = DeviceOverlay.from_rows(ov_ids, (rng.standard_normal((ov_ids.size, 128)) * 0.05).astype(np.float32),
                                 device=cuda)
    out_ov = tab.forward(torch.from_numpy(tokens), res, overlay=ov)
    got_ov = T.forward_rows([tab], rows, res, overlays=[ov])
    assert torch.equal(got_ov.view(torch.int16), out_ov.view(torch.int16))
    # an id outside the table: NaN in that head's 128 columns, the rest unchanged
    bad = rows.clone()
    bad[0, 5, 3] = 16 * 3000 + 7
    got_bad = T.forward_rows([tab], bad, res).float().cpu()
    assert torch.isnan(got_bad[5, 3 * 128:4 * 128]).all()
    ref = out.float().cpu()
    keep = torch.ones_like(ref, dtype=torch.bool)
    keep[5, 3 * 128:4 * 128] = False
    assert torch.equal(got_bad[keep], ref[keep])
    # two MXFP8 layers of 24 heads (2-, 3-, 4-grams)
    specs = [synthetic_spec(n_rows=24 * 3000, seed=126 + l, ngram_size=4) for l in range(2)]
    tabs = [G.device_table(specs[l], "mxfp8", 24 * 3000, 128, seed=128 + l) for l in range(2)]
    tok4 = synth.zipf_tokens(130, 1024, 129_280)
    res4 = G.residual(1024, 3072, seed=131)
    out4, rows4 = T.forward(tabs, torch.from_numpy(tok4), res4, return_rows=True)
    got4 = T.forward_rows(tabs, rows4, res4)
    assert torch.equal(got4.view(torch.int16), out4.view(torch.int16))


def test_stream_copy(cuda):
    """eg_stream_copy: byte-exact copies of several sizes; misaligned sizes refused."""
    from engraft_ngram_amd import table as T
    for n in (16, 4096 + 16, 3 * 1024 * 1024 + 48):
        src = torch.randint(0, 256, (n,), dtype=torch.uint8, device=cuda)
        dst = torch.zeros_like(src)
        T.stream_copy(src, dst)
        assert torch.equal(src, dst)
    with pytest.raises(ValueError):
        T.stream_copy(torch.zeros(20, dtype=torch.uint8, device=cuda), torch.zeros(20, dtype=torch.uint8, device=cuda))


def test_forward_config1_full_size(cuda):
    """BASELINE config 1 at its own size: 320,000,000-row Q8_0 table (43.5 GB),
    batch 8 x 2048 Zipf(1.1) tokens, residual [16384, 2048] bf16.  Every one of
    the 262,144 row ids is compared, and the whole output."""
    _say("forward cfg1 (43.5 GB table)")
    c = CFG1
    spec = synthetic_spec(n_rows=c["n_rows"], seed=200)
    tab = G.device_table(spec, "q8_0", c["n_rows"], c["dim"], seed=201)
    n = c["batch"] * c["seq"]
    tokens = synth.zipf_tokens(202, n, c["vocab"])
    res = G.residual(n, c["width"], seed=203)
    out, rows = tab.forward(torch.from_numpy(tokens), res, seq_len=c["seq"], return_rows=True)
    exp_rows, _, exp_out = FW.forward(spec, tokens, G.synth_fetch("q8_0", 201, 128), G.bf16_bits(res),
                                      seq_len=c["seq"])
    assert np.array_equal(rows[0].cpu().numpy(), exp_rows)
    G.assert_out_matches(G.bf16_bits(out), exp_out)
    # the highest rows of the table were generated too (64-bit index math)
    hi = np.arange(c["n_rows"] - 3, c["n_rows"])
    got_hi = tab.store.payload[hi].cpu().numpy()
    assert np.array_equal(got_hi, synth.synth_rows("q8_0", 201, hi, 128, 0.02)[0].view(np.uint8))
    del tab, out, rows, res
    torch.cuda.empty_cache()


def _q8_overlay(ids: np.ndarray, seed: int, dim: int = 128):
    """A seeded Q8_0 overlay store for sorted ``ids`` (row k = synthetic row k of
    ``seed``) and its oracle rows."""
    from engraft_ngram_amd import table as T
    from engraft_ngram_amd.overlay import DeviceOverlay
    store = T.RowStore.empty("q8_0", ids.size, dim, "cuda:0")
    T.fill_synthetic(store, seed=seed, sigma=0.02)
    ov = DeviceOverlay(torch.from_numpy(ids.astype(np.int32)).cuda(), store)
    return ov, (lambda k: synth.synth_dequant("q8_0", seed, np.asarray(k), dim, 0.02))


def _decode_expect(spec, tok2d, fetch, ov_ids, ov_fetch, res_bits):
    """Oracle of one decode step: each sequence hashed alone, its last position."""
    n_seq, ctx = tok2d.shape
    rows, emb, _ = FW.forward(spec, tok2d.reshape(-1), fetch, seq_len=ctx)
    rows, emb = rows[ctx - 1::ctx], emb[ctx - 1::ctx]
    hit = np.isin(ov_ids, rows)
    emb, _ = FW.substitute(emb, rows, ov_ids[hit], ov_fetch(np.flatnonzero(hit)))
    return rows, FW.residual_add(res_bits, [emb])


def test_decode_with_overlay_config3_shape(cuda):
    """BASELINE config 3's shape on a 1.6M-row table: 256 sequences x (2 context
    tokens + 1 new), a 500,000-row Q8_0 overlay resolved per id; the decode step
    equals the oracle and the full forward's last positions, by binary search
    and through the overlay's rank bitmap alike."""
    from engraft_ngram_amd import table as T
    c = CFG3
    spec = synthetic_spec(n_rows=16 * 100_000, seed=61)
    tab = G.device_table(spec, "q8_0", 16 * 100_000, 128, seed=62)
    rng = np.random.default_rng(63)
    ov_ids = np.sort(rng.choice(16 * 100_000, size=c["overlay_rows"], replace=False))
    ov, ov_fetch = _q8_overlay(ov_ids, seed=64)
    tok = synth.zipf_tokens(65, c["n_seq"] * c["ctx"], c["vocab"]).reshape(c["n_seq"], c["ctx"])
    tok[::7, 0] = 151_643  # some sequences open with EOS in their context
    res = G.residual(c["n_seq"], c["width"], seed=66)
    out, rows = T.forward_decode([tab], torch.from_numpy(tok), res, overlays=[ov], return_rows=True)
    exp_rows, exp_out = _decode_expect(spec, tok, G.synth_fetch("q8_0", 62, 128), ov_ids, ov_fetch,
                                       G.bf16_bits(res))
    assert np.array_equal(rows[0].cpu().numpy(), exp_rows)
    assert np.isin(exp_rows, ov_ids).any()  # the overlay was exercised
    G.assert_out_matches(G.bf16_bits(out), exp_out)
    # the same as the full forward over the flattened sequences, last positions
    res_full = torch.zeros((tok.size, c["width"]), dtype=torch.bfloat16, device=cuda)
    res_full[c["ctx"] - 1::c["ctx"]] = res
    full = tab.forward(torch.from_numpy(tok.reshape(-1)), res_full, overlay=ov, seq_len=c["ctx"])
    assert torch.equal(full[c["ctx"] - 1::c["ctx"]], out)
    # the overlay's rank bitmap in place of the binary search: the same bits
    from engraft_ngram_amd.overlay import DeviceOverlay
    ov_bm = DeviceOverlay(ov.ids, ov.rows).with_bitmap(tab.n_rows)
    out_bm, rows_bm = T.forward_decode([tab], torch.from_numpy(tok), res, overlays=[ov_bm], return_rows=True)
    assert torch.equal(out_bm, out) and torch.equal(rows_bm[0], rows[0])
    full_bm = tab.forward(torch.from_numpy(tok.reshape(-1)), res_full, overlay=ov_bm, seq_len=c["ctx"])
    assert torch.equal(full_bm, full)


def test_decode_config3_full_size(cuda):
    """BASELINE config 3 at its own size: the 320M-row config-1 table plus a
    500,000-row overlay, 256 sequences x 3 tokens."""
    from engraft_ngram_amd import table as T
    _say("decode cfg3 (43.5 GB table + 500k overlay)")
    c = CFG3
    spec = synthetic_spec(n_rows=c["n_rows"], seed=200)
    tab = G.device_table(spec, "q8_0", c["n_rows"], 128, seed=201)
    ov_ids = np.unique(np.random.default_rng(300).integers(0, c["n_rows"], size=c["overlay_rows"] + 2000))
    ov_ids = ov_ids[:c["overlay_rows"]]
    tok = synth.zipf_tokens(302, c["n_seq"] * c["ctx"], c["vocab"]).reshape(c["n_seq"], c["ctx"])
    rows_all = H.ngram_rows_np(spec, tok.reshape(-1), seq_len=c["ctx"])[c["ctx"] - 1::c["ctx"]]
    ov_ids = np.unique(np.concatenate([ov_ids[:-200], rows_all.reshape(-1)[:200]]))  # some ids are read
    ov, ov_fetch = _q8_overlay(ov_ids, seed=301)
    res = G.residual(c["n_seq"], c["width"], seed=303)
    out, rows = T.forward_decode([tab], torch.from_numpy(tok), res, overlays=[ov], return_rows=True)
    exp_rows, exp_out = _decode_expect(spec, tok, G.synth_fetch("q8_0", 201, 128), ov_ids, ov_fetch,
                                       G.bf16_bits(res))
    assert np.array_equal(rows[0].cpu().numpy(), exp_rows)
    G.assert_out_matches(G.bf16_bits(out), exp_out)
    # with the overlay's rank bitmap (81 MB over the 320M rows): the same bits
    from engraft_ngram_amd.overlay import DeviceOverlay
    ov_bm = DeviceOverlay(ov.ids, ov.rows).with_bitmap(c["n_rows"])
    out_bm = T.forward_decode([tab], torch.from_numpy(tok), res, overlays=[ov_bm])
    assert torch.equal(out_bm, out)
    del tab, ov, ov_bm
    torch.cuda.empty_cache()


def test_forward_config4_full_size(cuda):
    """BASELINE config 4 at its own size: 2 layers x 160,000,000 MXFP8 rows
    (42.2 GB), 2-/3-/4-gram hashes (24 slots per layer), 32,768 Zipf tokens over
    129,280, residual width 3,072.  Every row id is compared.  The rows the
    device gathers (eg_gather) equal the oracle's regenerated rows on 4,096
    sampled positions, and the whole output equals the oracle's fp32 residual
    add of the device-gathered rows at every position."""
    from engraft_ngram_amd import table as T
    _say("forward cfg4 (2 x 21 GB MXFP8 tables)")
    c = CFG4
    specs = [synthetic_spec(n_rows=c["n_rows"], seed=400 + l, ngram_size=4) for l in range(2)]
    tabs = [G.device_table(specs[l], "mxfp8", c["n_rows"], 128, seed=410 + l) for l in range(2)]
    tokens = synth.zipf_tokens(420, c["seq"], c["vocab"])
    res = G.residual(c["seq"], c["width"], seed=421)
    out, rows = T.forward(tabs, torch.from_numpy(tokens), res, return_rows=True)
    sample = np.sort(np.random.default_rng(422).choice(c["seq"], size=4096, replace=False))
    sample[:2] = [0, 1]  # the EOS-padded first positions
    embs, embs_all = [], []
    for l in range(2):
        r = H.ngram_rows_np(specs[l], tokens)
        assert np.array_equal(rows[l].cpu().numpy(), r)
        embs.append(FW.gather(r[sample], G.synth_fetch("mxfp8", 410 + l, 128)))
        dev_rows = tabs[l].gather(rows[l]).cpu().numpy()  # every position, through eg_gather
        assert np.array_equal(dev_rows[sample], embs[l])
        embs_all.append(dev_rows)
    got = G.bf16_bits(out)
    G.assert_out_matches(got[sample], FW.residual_add(G.bf16_bits(res)[sample], embs))
    G.assert_out_matches(got, FW.residual_add(G.bf16_bits(res), embs_all))
    del tabs, out, rows, res, embs_all
    torch.cuda.empty_cache()


def test_ple_table_from_gguf(cuda, tmp_path):
    """PleTable(path) on a per-head IQ4_NL GGUF (engraft/table.py:40-109): the
    hash parameters come from the metadata, read_rows_raw returns the file's
    bytes, read_rows their IQ4_NL dequantisation, ngram_addresses the scalar
    hash, and an all-zero-scale row reads as zero."""
    from engraft_ngram_amd import table as T
    from oracle import formats as F
    from tests.gguf_util import ple_table_file
    spec = fake_table_spec(5, head_vocab_size=300)
    rng = np.random.default_rng(1)
    raw = []
    for h in range(16):
        r = rng.integers(0, 256, size=(300, 90), dtype=np.uint8)
        for b in range(5):  # finite fp16 scales
            r[:, 18 * b:18 * b + 2] = np.frombuffer(
                (rng.standard_normal(300) * 1e-3).astype(np.float16).tobytes(), np.uint8).reshape(300, 2)
        raw.append(r)
    raw[4][17, [0, 1, 18, 19, 36, 37, 54, 55, 72, 73]] = 0  # row 17 of head 4: zero scales
    ple_table_file(tmp_path / "ple.gguf", spec, raw)
    tab = T.PleTable(tmp_path / "ple.gguf")
    assert isinstance(tab, T.PleTable) and isinstance(tab, T.DeviceTable) and tab.path == tmp_path / "ple.gguf"
    assert tab.head_offsets == list(spec.head_offsets) and tab.layer_multipliers == list(spec.layer_multipliers)
    assert tab.image_token_id == 151_655
    for h in (0, 4, 15):
        assert np.array_equal(tab.read_rows_raw(h, 10, 50), raw[h][10:60])
        np.testing.assert_array_equal(tab.read_rows(h, 10, 50), F.dequant_iq4nl(raw[h][10:60]))
    assert T.row_is_zero(tab.read_rows_raw(4, 17, 1))[0] and not tab.read_rows(4, 17, 1).any()
    tokens = [1, 2, 3, spec.eos_token_id, 9, 9]
    assert tab.ngram_addresses(tokens) == H.ngram_addresses_scalar(spec, tokens)
    with pytest.raises(AssertionError):
        tab.read_rows_raw(0, 299, 2)


def test_forward_graph_capture_replays(cuda):
    """A PreparedForward captured in a HIP graph: three replays with the
    program's own eager work between them (a new residual written in place, an
    eager forward of the same inputs), every replay equal to the eager result
    and to the oracle.  The forward records no memset."""
    from engraft_ngram_amd import table as T
    from engraft_ngram_amd.overlay import DeviceOverlay
    _say("graph capture of the forward")
    spec = synthetic_spec(n_rows=16 * 2000, seed=61)
    tab = G.device_table(spec, "q8_0", 16 * 2000, 128, seed=62)
    tokens = synth.zipf_tokens(63, 2048, 5000)
    rows = H.ngram_rows_np(spec, tokens)
    rng = np.random.default_rng(64)
    ov_ids = np.unique(rng.choice(np.unique(rows), size=200, replace=False)).astype(np.int32)
    ov_rows = (rng.standard_normal((ov_ids.size, 128)) * 0.05).astype(np.float32)
    ov = DeviceOverlay.from_rows(ov_ids, ov_rows, device=cuda)
    tok = torch.from_numpy(tokens).to(cuda)
    res = G.residual(tokens.size, 2048, seed=65)
    out = torch.empty_like(res)
    call = T.PreparedForward([tab], tok, res, out=out, overlays=[ov], seq_len=1024)
    side = torch.cuda.Stream(cuda)
    side.wait_stream(torch.cuda.current_stream(cuda))
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream(cuda).wait_stream(side)
    torch.cuda.synchronize(cuda)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    fetch = G.synth_fetch("q8_0", 62, 128)
    for k in range(3):
        res.copy_(G.residual(tokens.size, 2048, seed=70 + k))
        eager = tab.forward(tok, res, overlay=ov, seq_len=1024)
        torch.cuda.synchronize(cuda)
        out.zero_()
        g.replay()
        torch.cuda.synchronize(cuda)
        assert torch.equal(out, eager), f"replay {k}"
        _, _, exp = FW.forward(spec, tokens, fetch, G.bf16_bits(res), overlay=(ov_ids, ov_rows), seq_len=1024)
        G.assert_out_matches(G.bf16_bits(out), exp)


def test_mxfp8_every_code_decodes_exactly(cuda):
    """Every e4m3 code (0..255) under e8m0 scales 2^0, 2^-7, 2^7 and 2^-126 (the
    last giving subnormal products), through eg_gather -- gfx950's packed fp8
    conversion -- against the oracle's definition of the format: bit-exact,
    and NaN exactly where the code is 0x7f or 0xff."""
    _say("mxfp8 every code")
    spec = synthetic_spec(n_rows=16, seed=3)  # 16 heads of one row each
    codes = np.arange(256, dtype=np.uint8).reshape(2, 128)
    payload = np.zeros((16, 128), dtype=np.uint8)
    scales = np.full((16, 4), 127, dtype=np.uint8)
    for i, e in enumerate((127, 120, 134, 1)):
        payload[2 * i:2 * i + 2] = codes
        scales[2 * i:2 * i + 2] = e
    tab = G.table_from_arrays(spec, "mxfp8", 128, payload, scales)
    got = tab.gather(torch.arange(16, dtype=torch.int32).reshape(-1, 1)).cpu().numpy()
    exp = G.F.dequant_mxfp8(payload, scales)
    nan = np.isnan(exp)
    assert nan.sum() == 4 * 2 and np.array_equal(np.isnan(got), nan)  # 0x7f and 0xff per scale
    assert np.array_equal(got[~nan].view(np.uint32), exp[~nan].view(np.uint32))


def test_forward_edge_cases(cuda):
    """Empty input; one-token and ragged segments (the hash substitutes EOS for
    missing predecessors and never looks across a segment start); a last
    sequence shorter than seq_len; the residual updated in place."""
    from engraft_ngram_amd import table as T
    _say("forward edge cases")
    spec = synthetic_spec(n_rows=16 * 1000, seed=91)
    tab = G.device_table(spec, "q8_0", 16 * 1000, 128, seed=92)
    fetch = G.synth_fetch("q8_0", 92, 128)
    empty = tab.forward(torch.zeros(0, dtype=torch.int64), torch.zeros((0, 2048), dtype=torch.bfloat16, device=cuda))
    assert empty.shape == (0, 2048)
    rng = np.random.default_rng(93)
    tokens = rng.integers(0, 40, size=37)
    # ragged segments, including single-token ones
    starts = np.array([0, 1, 2, 9, 10, 30, 36])
    seg_start = np.zeros(37, dtype=np.int32)
    for s in starts:
        seg_start[s:] = s
    res = G.residual(37, 2048, seed=94)
    out = tab.forward(torch.from_numpy(tokens), res, seg_start=torch.from_numpy(seg_start))
    _, _, exp = FW.forward(spec, tokens, fetch, G.bf16_bits(res), seg_start=seg_start)
    G.assert_out_matches(G.bf16_bits(out), exp)
    # seq_len 16 over 37 positions: the last sequence holds 5
    out = tab.forward(torch.from_numpy(tokens), res, seq_len=16)
    _, _, exp = FW.forward(spec, tokens, fetch, G.bf16_bits(res), seq_len=16)
    G.assert_out_matches(G.bf16_bits(out), exp)
    # in place: out is the residual
    res2 = res.clone()
    T.forward([tab], torch.from_numpy(tokens), res2, out=res2, seq_len=16)
    assert torch.equal(res2, out)


def test_forward_on_two_streams(cuda):
    """Calls on different streams are independent: two batches launched on two
    non-default streams (default priority) give the results of the same calls
    made one after the other on the default stream."""
    _say("forward on two streams")
    spec = synthetic_spec(n_rows=16 * 2000, seed=111)
    tab = G.device_table(spec, "q8_0", 16 * 2000, 128, seed=112)
    toks = [torch.from_numpy(synth.zipf_tokens(113 + k, 4096, 5000)) for k in range(2)]
    res = [G.residual(4096, 2048, seed=115 + k) for k in range(2)]
    exp = [tab.forward(toks[k], res[k], seq_len=1024) for k in range(2)]
    torch.cuda.synchronize(cuda)
    streams = [torch.cuda.Stream(cuda) for _ in range(2)]
    got = [None, None]
    for k in range(2):
        streams[k].wait_stream(torch.cuda.current_stream(cuda))
        with torch.cuda.stream(streams[k]):
            got[k] = tab.forward(toks[k], res[k], seq_len=1024)
    torch.cuda.synchronize(cuda)
    for k in range(2):
        assert torch.equal(got[k], exp[k])


def test_iq4nl_rows_in_padded_lines(cuda, tmp_path):
    """IQ4_NL rows each in a 128-byte line (PleTable's default): the forward,
    the gather, the raw and dequantised row reads and the hash match the same
    table in its packed 90-byte rows bit for bit; the C boundary refuses a
    stride for another format or an odd one."""
    import ctypes

    from engraft_ngram_amd import _lib
    from engraft_ngram_amd import table as T
    from tests.gguf_util import ple_table_file
    spec = fake_table_spec(7, head_vocab_size=400)
    assert list(spec.head_offsets) == [400 * h for h in range(16)]
    rng = np.random.default_rng(2)
    raw = []
    for h in range(16):
        r = rng.integers(0, 256, size=(400, 90), dtype=np.uint8)
        for b in range(5):
            r[:, 18 * b:18 * b + 2] = np.frombuffer(
                (rng.standard_normal(400) * 1e-3).astype(np.float16).tobytes(), np.uint8).reshape(400, 2)
        raw.append(r)
    ple_table_file(tmp_path / "ple.gguf", spec, raw)
    padded = T.PleTable(tmp_path / "ple.gguf")
    packed = T.PleTable(tmp_path / "ple.gguf", pad_rows=False, chunk_bytes=90 * 7)
    assert padded.store.row_stride == 128 and tuple(padded.store.payload.shape)[1] == 128
    assert packed.store.row_stride == 0 and tuple(packed.store.payload.shape)[1] == 90
    for h in (0, 9, 15):
        assert np.array_equal(padded.read_rows_raw(h, 3, 100), raw[h][3:103])
        assert np.array_equal(packed.read_rows_raw(h, 3, 100), raw[h][3:103])
        assert np.array_equal(padded.read_rows(h, 3, 100), packed.read_rows(h, 3, 100))
    tokens = synth.zipf_tokens(3, 4096, 6000)
    res = G.residual(tokens.size, 16 * 160, seed=4)
    a = padded.forward(torch.from_numpy(tokens), res, seq_len=1024)
    b = packed.forward(torch.from_numpy(tokens), res, seq_len=1024)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    rows = padded.rows(torch.from_numpy(tokens), seq_len=1024)
    assert torch.equal(padded.gather(rows), packed.gather(rows))
    fetch = lambda ids: G.F.dequant_iq4nl(np.concatenate(raw)[np.asarray(ids).reshape(-1)])  # noqa: E731
    _, _, exp = FW.forward(spec, tokens[:512], fetch, G.bf16_bits(res[:512]), seq_len=1024)
    G.assert_out_matches(G.bf16_bits(a[:512]), exp)
    # the boundary's checks (host side, before any launch)
    q8 = T.RowStore.empty("q8_0", 16, 128, cuda).c_table()
    q8.row_stride = 256
    out = torch.empty((1, 128), dtype=torch.float32, device=cuda)
    one = torch.zeros((1, 1), dtype=torch.int32, device=cuda)
    rc = _lib.load().eg_gather(ctypes.byref(q8), None, _lib.ptr(one), 1, 1, _lib.ptr(out), _lib.stream_ptr(cuda))
    assert rc == _lib.EG_ERR_ARG
    odd = padded.store.c_table()
    odd.row_stride = 127
    rc = _lib.load().eg_gather(ctypes.byref(odd), None, _lib.ptr(one), 1, 1, _lib.ptr(out), _lib.stream_ptr(cuda))
    assert rc == _lib.EG_ERR_ARG


def test_forward_slots_two_layers_with_overlays(cuda):
    """eg_forward_slots over two table layers, each with its own overlay (one
    with an index into a larger store): per layer, every slot's overlay row
    (the index entry, or the id's rank) or -1, as the oracle's search finds
    it; the output equals eg_forward's bit for bit."""
    from engraft_ngram_amd import table as T
    from engraft_ngram_amd.overlay import DeviceOverlay
    specs = [synthetic_spec(n_rows=16 * 3000, seed=131 + l) for l in range(2)]
    tabs = [G.device_table(specs[l], "q8_0", 16 * 3000, 128, seed=133 + l) for l in range(2)]
    tokens = synth.zipf_tokens(135, 2048, 4000)
    rng = np.random.default_rng(136)
    ovs, exp = [], []
    for l in range(2):
        rows = H.ngram_rows_np(specs[l], tokens, seq_len=1024)
        ids = np.unique(rng.choice(np.unique(rows), size=400, replace=False)).astype(np.int32)
        vals = (rng.standard_normal((ids.size, 128)) * 0.05).astype(np.float32)
        if l == 0:
            ov = DeviceOverlay.from_rows(ids, vals, device=cuda)
            slot_row = np.arange(ids.size)
        else:
            # an index into a store with the rows in reverse order
            store_rows = torch.from_numpy(vals[::-1].copy()).to(cuda)
            index = np.arange(ids.size)[::-1].astype(np.int32).copy()
            ov = DeviceOverlay(torch.from_numpy(ids).to(cuda), T.RowStore("f32", 128, store_rows),
                               index=torch.from_numpy(index).to(cuda))
            slot_row = index
        pos = np.searchsorted(ids, rows)
        hit = (pos < ids.size) & (ids[np.minimum(pos, ids.size - 1)] == rows)
        exp.append(np.where(hit, slot_row[np.minimum(pos, ids.size - 1)], -1))
        ovs.append(ov)
    res = G.residual(tokens.size, 2048, seed=137)
    call = T.PreparedForward(tabs, torch.from_numpy(tokens), res, overlays=ovs, seq_len=1024,
                             return_slot_vars=True)
    call()
    plain = T.forward(tabs, torch.from_numpy(tokens), res, overlays=ovs, seq_len=1024)
    torch.cuda.synchronize()
    sv = call.slot_vars.cpu().numpy()
    for l in range(2):
        assert np.array_equal(sv[l], exp[l]), l
    assert (sv >= 0).any() and (sv == -1).any()
    assert torch.equal(call.out.view(torch.int16), plain.view(torch.int16))


@pytest.mark.parametrize("fmt", ["q8_0", "bf16", "f32", "iq4_nl", "mxfp8"])
def test_dequant_wire_blocks_against_oracle(cuda, fmt):
    """eg_dequant_blocks (the dequant_q8_0 / dequant_bf16 / dequant_iq4_nl /
    dequant_f32 drop-ins, engraft/replica/dequant.py:71-147) on every byte
    pattern of random blocks, against the oracle's wire decode (bit-exact;
    NaN where the oracle has NaN); then read_rows_raw's wire form of a device
    table decoded by the drop-in equals read_rows."""
    from engraft_ngram_amd import _lib, dequant
    from oracle import formats as F
    print(f"[gpu-test] dequant wire blocks {fmt}", flush=True)
    bb = F.WIRE_BLOCK_BYTES[fmt]
    raw = np.random.default_rng(3).integers(0, 256, (1000 * 3 + 7, bb)).astype(np.uint8)
    want = F.dequant_wire(fmt, raw)
    if fmt == "mxfp8":
        out = torch.empty((raw.shape[0], 32), dtype=torch.float32, device=cuda)
        src = torch.as_tensor(raw, device=cuda)
        _lib.call("eg_dequant_blocks", _lib.FMT_CODES[fmt], _lib.ptr(src), raw.shape[0], _lib.ptr(out),
                  _lib.stream_ptr(cuda))
        got = out.cpu().numpy()
    else:
        fn = dequant.DEQUANT_FNS[fmt.upper()]
        got = fn(torch.as_tensor(raw, device=cuda).reshape(1000 * 3 + 7, bb)).cpu().numpy()
        # a CPU tensor comes back on the CPU; out_dtype as the reference's .to()
        fin = np.flatnonzero(np.isfinite(want).all(axis=1))[:5]
        cpu_in = torch.as_tensor(raw[fin].reshape(5, 1, bb))
        back = fn(cpu_in, out_dtype=torch.bfloat16)
        assert back.device.type == "cpu" and back.dtype == torch.bfloat16 and back.shape[:2] == (5, 1)
        assert torch.equal(back.reshape(5, -1), torch.as_tensor(want[fin]).to(torch.bfloat16))
        with pytest.raises(AssertionError):
            fn(torch.zeros((2, bb + 1), dtype=torch.uint8, device=cuda))
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    if fmt in ("q8_0", "bf16"):
        spec = synthetic_spec(n_rows=16 * 300, seed=4)
        tab = G.device_table(spec, fmt, 16 * 300, 128, seed=5)
        raw_rows = tab.read_rows_raw(3, 17, 40)
        fn = dequant.DEQUANT_FNS[fmt.upper()]
        dec = fn(torch.from_numpy(raw_rows).reshape(40, -1, bb)).reshape(40, -1).numpy()
        assert np.array_equal(dec, tab.read_rows(3, 17, 40))


def test_stream_ptr_is_the_current_stream(cuda):
    """``_lib.stream_ptr`` (torch's raw-stream query) names the stream torch
    calls current, for every way of giving the device and inside a stream
    context: the launches go where torch's own work goes."""
    from engraft_ngram_amd import _lib

    _say("stream_ptr")
    dev = torch.device("cuda", torch.cuda.current_device())
    forms = (None, dev, dev.index, f"cuda:{dev.index}", torch.device("cuda"))
    want = int(torch.cuda.current_stream(dev).cuda_stream)
    assert all(_lib.stream_ptr(d) == want for d in forms)
    s = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(s):
        assert int(s.cuda_stream) != want
        assert all(_lib.stream_ptr(d) == int(s.cuda_stream) for d in forms)
    assert _lib.stream_ptr(dev) == want
