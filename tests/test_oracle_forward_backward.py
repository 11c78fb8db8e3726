"""Pins the CPU oracle's gather/substitution/residual add and its scatter/Adam
(no GPU)."""
from __future__ import annotations

import math

import numpy as np
import torch

from oracle import backward as B
from oracle import formats as F
from oracle import forward as FW
from oracle import hash as H
from oracle import synth
from tests.params import fake_table_spec


def _small_table(spec, dim=128, seed=3):
    n_rows = spec.head_offsets[-1] + spec.head_vocab_sizes[-1]
    payload, scales = synth.synth_rows("q8_0", seed, np.arange(n_rows), dim, 0.02)
    return FW.table_fetch("q8_0", payload, scales)


def test_gather_equals_per_position_rowset_loop():
    """engraft/lens.py:126-136: per position, rows_global[h] = offset + local and
    data[h] = read_rows(h, local, 1)."""
    spec = fake_table_spec(2, head_vocab_size=300)
    fetch = _small_table(spec)
    tokens = [5, 9, 9, 2, spec.eos_token_id, 7, 1]
    rows = H.ngram_rows_np(spec, tokens)
    emb = FW.gather(rows, fetch)
    addr = H.ngram_addresses_scalar(spec, tokens)
    for t in range(len(tokens)):
        for h in range(spec.n_heads):
            g = H.local_to_global(spec, h, addr[t][h])
            assert rows[t, h] == g
            np.testing.assert_array_equal(emb[t, h * 128:(h + 1) * 128], fetch(np.array([g]))[0])


def test_overlay_substitutes_present_rows_only():
    """tests/test_replica_graft.py:43-70: a row present in the overlay is replaced,
    every other head bit-identical; an empty overlay is the plain gather."""
    spec = fake_table_spec(7, head_vocab_size=300)
    fetch = _small_table(spec)
    tokens = [1, 2, 3, 4, 5]
    rows = H.ngram_rows_np(spec, tokens)
    base = FW.gather(rows, fetch)
    g0 = int(rows[3, 0])
    vec = np.full((1, 128), 99.0, dtype=np.float32)
    out, hits = FW.substitute(base, rows, np.array([g0]), vec)
    assert hits == int((rows == g0).sum()) >= 1
    o3 = out.reshape(5, 16, 128)
    b3 = base.reshape(5, 16, 128)
    for t in range(5):
        for h in range(16):
            if rows[t, h] == g0:
                assert np.array_equal(o3[t, h], vec[0])
            else:
                assert np.array_equal(o3[t, h], b3[t, h])
    same, hits0 = FW.substitute(base, rows, np.array([], dtype=np.int64), np.zeros((0, 128), np.float32))
    assert hits0 == 0 and np.array_equal(same, base)


def test_residual_add_is_fp32_add_then_bf16_rne():
    """bf16_rne(f32(res) + e0 + e1) against torch's fp32 add and bf16 cast."""
    rng = np.random.default_rng(0)
    res = torch.randn(64, 256, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    e0 = rng.standard_normal((64, 256)).astype(np.float32) * 0.02
    e1 = rng.standard_normal((64, 256)).astype(np.float32) * 0.02
    got = FW.residual_add(res.view(torch.int16).numpy().view(np.uint16), [e0, e1])
    ref = ((res.float() + torch.from_numpy(e0)) + torch.from_numpy(e1)).to(torch.bfloat16)
    assert np.array_equal(got, ref.view(torch.int16).numpy().view(np.uint16))


def test_scatter_grad_against_exact_sum_and_order():
    rng = np.random.default_rng(1)
    p, hh, d = 300, 16, 32
    # many duplicates; heads 8..15 draw from 4 rows only: segments of ~75 slots
    rows = rng.integers(0, 40, size=(p, hh))
    rows[:, 8:] %= 4
    rows = rows + np.arange(hh)[None, :] * 40
    ids = np.unique(rows)[::2]  # half of the rows are variables
    d_emb = (rng.standard_normal((p, hh * d)) * 1e-3).astype(np.float32)
    grad, hits = B.scatter_grad(d_emb, rows, ids)
    exact = B.scatter_grad_exact(d_emb, rows, ids)
    assert hits.sum() == np.isin(rows, ids).sum()
    # sequential fp32 summation error bound: n * eps * sum|x|
    absum = B.scatter_grad_exact(np.abs(d_emb), rows, ids)
    bound = hits[:, None] * np.finfo(np.float32).eps * absum + 1e-30
    assert np.all(np.abs(grad - exact) <= bound)
    # segments of at most 32 slots: ascending slot order, one addition at a
    # time -- a manual loop reproduces them bit for bit
    keys = B.slot_keys(rows, ids)
    manual = np.zeros_like(grad)
    for s in range(p * hh):
        if keys[s] >= 0:
            manual[keys[s]] += d_emb.reshape(p * hh, d)[s]
    short = hits <= B.PIECE
    assert short.any() and (~short).any()
    assert np.array_equal(manual[short], grad[short])


def test_segment_sum_long_association():
    """Long segments: pieces of 32 summed in order, piece j added to group j % 8,
    groups added in order -- restated here with reshapes and cumsum."""
    rng = np.random.default_rng(6)
    for n in (33, 64, 255, 256, 257, 1000, 5000):
        x = (rng.standard_normal((n, 16)) * 1e-3).astype(np.float32)
        pad = (-n) % 32
        xp = np.concatenate([x, np.zeros((pad, 16), np.float32)])
        pieces = []
        for blk in xp.reshape(-1, 32, 16):
            acc = np.zeros(16, np.float32)
            for r in blk:  # trailing zero rows do not change an fp32 sum
                acc = np.float32(acc + r)
            pieces.append(acc)
        groups = [np.zeros(16, np.float32) for _ in range(8)]
        for j, pc in enumerate(pieces):
            groups[j % 8] = np.float32(groups[j % 8] + pc)
        tot = groups[0]
        for g in groups[1:]:
            tot = np.float32(tot + g)
        assert np.array_equal(B.segment_sum(x), tot)
        assert np.allclose(B.segment_sum(x), x.astype(np.float64).sum(0), rtol=0, atol=1e-6)


def test_adam_dense_matches_torch_adam_multistep():
    """engraft/descend_corpus.py:790,947: torch.optim.Adam([rows_var], lr)."""
    rng = np.random.default_rng(2)
    p0 = (rng.standard_normal((50, 128)) * 0.02).astype(np.float32)
    grads = [(rng.standard_normal((50, 128)) * 1e-3).astype(np.float32) for _ in range(4)]
    grads[2][::3] = 0.0
    t = torch.from_numpy(p0.copy()).requires_grad_(True)
    opt = torch.optim.Adam([t], lr=1e-3, betas=(0.9, 0.999), eps=1e-8)
    p, m, v = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    for k, g in enumerate(grads, start=1):
        opt.zero_grad()
        t.grad = torch.from_numpy(g.copy())
        opt.step()
        p, m, v = B.adam_step(p, g, m, v, k, 1e-3)
        ref = t.detach().numpy()
        assert np.max(np.abs(p - ref)) <= 1e-6 * np.max(np.abs(ref))


def test_adam_first_step_closed_form():
    """m_hat = g, v_hat = g**2 on step 1: p1 = p0 - lr * g / (|g| + eps)."""
    rng = np.random.default_rng(3)
    p0 = (rng.standard_normal((20, 64)) * 0.02).astype(np.float32)
    g = (rng.standard_normal((20, 64)) * 1e-3).astype(np.float32)
    p1, m, v = B.adam_step(p0, g, np.zeros_like(p0), np.zeros_like(p0), 1, 1e-3)
    closed = p0.astype(np.float64) - 1e-3 * g / (np.abs(g) + 1e-8)
    np.testing.assert_allclose(p1, closed, rtol=0, atol=1e-8)  # ~2 fp32 ulps at |p| ~ 0.05
    np.testing.assert_allclose(m, 0.1 * g, rtol=1e-6)
    np.testing.assert_allclose(v, 0.001 * g.astype(np.float64) ** 2, rtol=1e-5)


def test_adam_sparse_leaves_untouched_rows():
    rng = np.random.default_rng(4)
    p0 = rng.standard_normal((10, 8)).astype(np.float32)
    m0 = rng.standard_normal((10, 8)).astype(np.float32) * 1e-3
    v0 = np.abs(rng.standard_normal((10, 8)).astype(np.float32)) * 1e-6
    g = rng.standard_normal((10, 8)).astype(np.float32)
    touched = np.zeros(10, dtype=bool)
    touched[[1, 4, 7]] = True
    p1, m1, v1 = B.adam_step(p0, g, m0, v0, 3, 1e-3, touched=touched)
    pd, md, vd = B.adam_step(p0, g, m0, v0, 3, 1e-3)
    assert np.array_equal(p1[~touched], p0[~touched]) and np.array_equal(m1[~touched], m0[~touched])
    assert np.array_equal(p1[touched], pd[touched]) and np.array_equal(v1[touched], vd[touched])
    assert math.isclose(float(np.abs(p1 - p0).max()), float(np.abs(pd[touched] - p0[touched]).max()))


def test_cpu_baseline_equals_oracle_forward():
    """bench.py's cpu_baseline leg computes the same bits as oracle.forward, in
    both its vectorized and its literal per-position form."""
    from oracle import cpu_baseline as CB
    from tests.params import synthetic_spec

    spec = synthetic_spec(n_rows=16 * 3000, seed=12)
    tokens = synth.zipf_tokens(13, 2 * 256, 151_936)
    host = CB.HostTable(16 * 3000, 128)
    rows0 = H.ngram_rows_np(spec, tokens, seq_len=256)
    host.populate(14, rows0)
    res = torch.randn(512, 2048, generator=torch.Generator().manual_seed(15)).to(torch.bfloat16)
    rows, out = CB.forward_q8(spec, tokens, 256, host, res)
    fetch = FW.table_fetch("q8_0", host.payload, host.scales)
    exp_rows, _, exp_out = FW.forward(spec, tokens, fetch, res.view(torch.int16).numpy().view(np.uint16),
                                      seq_len=256)
    assert np.array_equal(rows, exp_rows)
    assert np.array_equal(out.view(torch.int16).numpy().view(np.uint16), exp_out)
    # the literal per-position loop (scalar re-hash of every prefix) gives the same bits
    lit = CB.forward_q8_literal(spec, tokens, 40, host, res[:40].view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(lit, exp_out[:40])
    # the format-generic form with a row reader gives the same bits
    read = lambda r: FW.table_fetch("q8_0", host.payload, host.scales)(np.array([r]))[0]
    lit2 = CB.forward_literal(spec, tokens, 40, read, 128, res[:40].view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(lit2, exp_out[:40])


def test_product_synthetic_params_equal_oracle_params():
    """The benchmark's synthetic addressing (engraft_ngram_amd.synthetic) is the
    one the parity tests use (tests.params.synthetic_spec)."""
    from engraft_ngram_amd import synthetic as S
    from tests.params import synthetic_spec

    for ng in (3, 4):
        spec = synthetic_spec(n_rows=320_000_000, seed=200, ngram_size=ng)
        hp = S.hash_params(320_000_000, 200, ngram_size=ng)
        assert tuple(hp["head_vocab_sizes"]) == spec.head_vocab_sizes
        assert tuple(hp["head_offsets"]) == spec.head_offsets
        assert tuple(tuple(r) for r in hp["head_multipliers"]) == spec.head_multipliers
        assert hp["eos_token_id"] == spec.eos_token_id
    assert np.array_equal(S.zipf_tokens(5, 1000, 151_936), synth.zipf_tokens(5, 1000, 151_936))


def test_adam_pull_term_matches_torch_autograd():
    """The pull term of engraft/descend_corpus.py:935-939 through torch autograd
    + torch.optim.Adam on CPU, three dense steps."""
    rng = np.random.default_rng(5)
    rows0 = (rng.standard_normal((30, 128)) * 0.02).astype(np.float32)
    mu = 0.1
    t = torch.from_numpy(rows0.copy()).requires_grad_(True)
    r0t = torch.from_numpy(rows0.copy())
    opt = torch.optim.Adam([t], lr=1e-3)
    p, m, v = rows0.copy(), np.zeros_like(rows0), np.zeros_like(rows0)
    s = np.float32((rows0.astype(np.float32) ** 2).sum(dtype=np.float32))
    coef = float(np.float32(mu) / s)
    for k in range(1, 4):
        g = (rng.standard_normal((30, 128)) * 1e-3).astype(np.float32)
        opt.zero_grad()
        t.grad = torch.from_numpy(g.copy())
        reg = mu * ((t - r0t).pow(2).sum() / r0t.pow(2).sum().clamp_min(1e-12))
        reg.backward()
        opt.step()
        p, m, v = B.adam_step(p, g, m, v, k, 1e-3, rows0=rows0, l2_coef=coef)
        ref = t.detach().numpy()
        assert np.max(np.abs(p - ref)) <= 1e-6 * np.max(np.abs(ref))
