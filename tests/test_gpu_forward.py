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
from tests.params import CFG0, CFG1, fake_table_spec, reference_corpus, synthetic_spec, tiny_hparams_spec

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
