"""GPU parity of the descent backward: the deterministic scatter (sort +
segmented reduce) and the optimizer step + requantisation.

Bar: gradients bit-exact against the oracle's sequential ascending-slot fp32
sum; overlay rows after a step within 1e-5 relative of the oracle (asserted
bit-exact too: the step is IEEE fp32 in the same order); requantised rows
bit-exact against the oracle's rule applied to the device's fp32 rows; two runs
from the same state bitwise identical."""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import backward as B
from oracle import formats as F
from oracle import forward as FW
from oracle import hash as H
from oracle import synth
from tests import gpu_util as G
from tests.params import CFG1, synthetic_spec

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


def _rel_ok(got: np.ndarray, exp: np.ndarray, tol: float = 1e-5) -> float:
    """max |got - exp| / max |exp| per row (the 1e-5 relative bar)."""
    scale = np.maximum(np.abs(exp).max(axis=1, keepdims=True), 1e-30)
    rel = float((np.abs(got - exp) / scale).max()) if got.size else 0.0
    assert rel <= tol, f"relative error {rel}"
    return rel


@pytest.mark.parametrize("f32_grad", [False, True])
def test_scatter_grad_bit_exact(cuda, f32_grad):
    from engraft_ngram_amd import descent as D
    spec = synthetic_spec(n_rows=16 * 3000, seed=61)
    tokens = synth.zipf_tokens(62, 3000, 2000)  # many repeated bigrams -> long segments
    rows = H.ngram_rows_np(spec, tokens)
    uniq = np.unique(rows)
    ids = uniq[::2].astype(np.int32)  # half of the rows are variables, the rest frozen
    g = torch.Generator(device=cuda).manual_seed(63)
    d = torch.randn((3000, 2048), generator=g, device=cuda) * 1e-3
    d = d if f32_grad else d.to(torch.bfloat16)
    grad = D.scatter_grad(d, torch.from_numpy(rows.astype(np.int32)), torch.from_numpy(ids), 128).cpu().numpy()
    d_np = d.float().cpu().numpy()
    exp, hits = B.scatter_grad(d_np, rows, ids)
    assert hits.max() > 50  # a long segment was exercised
    assert np.array_equal(grad, exp)
    # repeatable, and accumulates into a given buffer
    again = D.scatter_grad(d, torch.from_numpy(rows.astype(np.int32)), torch.from_numpy(ids), 128,
                           grad=torch.from_numpy(grad).to(cuda)).cpu().numpy()
    assert np.array_equal(again, (grad + exp).astype(np.float32))


def test_scatter_grad_edge_cases(cuda):
    """Empty batch, no variable hit, a single variable hit by every position."""
    from engraft_ngram_amd import descent as D
    ids = torch.tensor([5, 9], dtype=torch.int32)
    d = torch.ones((0, 128), device=cuda)
    assert D.scatter_grad(d, torch.zeros((0, 1), dtype=torch.int32), ids, 128).abs().sum().item() == 0
    rows = torch.full((70, 1), 7, dtype=torch.int32)
    d = torch.randn((70, 128), device=cuda)
    assert D.scatter_grad(d, rows, ids, 128).abs().sum().item() == 0
    # one variable hit by every slot: ordered in LDS (5,000 slots) and, past the
    # LDS capacity of 8,192 slot ids, on global memory (20,000 slots)
    for n in (5000, 20000):
        rows = torch.full((n, 1), 9, dtype=torch.int32)
        d = torch.randn((n, 128), device=cuda)
        got = D.scatter_grad(d, rows, ids, 128).cpu().numpy()
        exp, _ = B.scatter_grad(d.cpu().numpy(), rows.numpy(), ids.numpy())
        assert np.array_equal(got, exp)


@pytest.mark.parametrize("n_slots,n_var,heads,dim,f32", [(30_000, 9_000, 16, 128, True), (20_500, 40, 1, 64, False),
                                                         (300_000, 3_000_000, 4, 160, True)],
                         ids=["overlay-emb-shape", "long-ranges", "counting-grouping"])
def test_scatter_grad_plan_apply_matches_one_call(cuda, n_slots, n_var, heads, dim, f32):
    """eg_scatter_grad_plan_slots + eg_scatter_grad_apply against
    eg_scatter_grad_slots, bit for bit: overwrite (every variable written,
    zeros where no slot reads it) and accumulate, the grouping applied twice
    (the second apply sees ranges the first ordered in place: a variable of
    18,000 slots, past the 4,096 ordered in LDS), bf16 and f32 gradients;
    an empty batch with overwrite writes zeros."""
    from engraft_ngram_amd import _lib
    _say(f"scatter plan/apply, {n_slots} slots over {n_var} variables, heads {heads}, dim {dim}")
    rng = np.random.default_rng(5)
    n_pos = n_slots // heads
    sv = ((rng.zipf(1.3, size=n_pos * heads) - 1) % (n_var + n_var // 10)).astype(np.int32)  # some past n_var
    sv[rng.random(sv.size) < 0.1] = -1
    if n_var == 40:
        sv[:18_000] = 3  # one variable of 18,000 slots
    sv[sv == n_var - 1] = -1  # the last variable: no slot reads it
    slot_var = torch.from_numpy(sv.reshape(n_pos, heads)).to(cuda)
    d = torch.randn((n_pos, heads * dim), device=cuda)
    if not f32:
        d = d.to(torch.bfloat16)
    fl = 1 if f32 else 0
    st = _lib.stream_ptr(cuda)
    need = int(_lib.load().eg_backward_workspace_size(n_pos * heads, n_var))
    ws1 = torch.empty(need, dtype=torch.uint8, device=cuda)
    ref = torch.zeros((n_var, dim), device=cuda)
    _lib.call("eg_scatter_grad_slots", _lib.ptr(d), fl, _lib.ptr(slot_var), n_pos, heads, dim, n_var, _lib.ptr(ref),
              _lib.ptr(ws1), need, st)
    ws = torch.empty(need, dtype=torch.uint8, device=cuda)
    _lib.call("eg_scatter_grad_plan_slots", _lib.ptr(slot_var), n_pos, heads, n_var, _lib.ptr(ws), need, st)
    for rep in range(2):
        got = torch.full((n_var, dim), float("nan"), device=cuda)
        _lib.call("eg_scatter_grad_apply", _lib.ptr(d), fl, n_pos, heads, dim, n_var, _lib.ptr(got), 1, _lib.ptr(ws),
                  need, st)
        assert torch.equal(got.view(torch.int32), ref.view(torch.int32)), rep
    acc = torch.ones((n_var, dim), device=cuda)
    _lib.call("eg_scatter_grad_apply", _lib.ptr(d), fl, n_pos, heads, dim, n_var, _lib.ptr(acc), 0, _lib.ptr(ws),
              need, st)
    assert torch.equal(acc, 1.0 + ref)
    hit = np.bincount(sv[(sv >= 0) & (sv < n_var)], minlength=n_var)
    assert (hit == 0).any() and bool((ref[torch.from_numpy(hit == 0).to(cuda)] == 0).all())
    empty = torch.full((n_var, dim), float("nan"), device=cuda)
    _lib.call("eg_scatter_grad_apply", None, fl, 0, heads, dim, n_var, _lib.ptr(empty), 1, None, 0, st)
    assert bool((empty == 0).all())


@pytest.mark.parametrize("n_slots,n_var", [(1_100_000, 300_000), (1_000_000, 1_500_000), (400_000, 100_000)],
                         ids=["counting-1075-tiles", "buckets-of-2048-variables", "buckets-391-tiles"])
def test_scatter_grad_large_groupings(cuda, n_slots, n_var):
    """The two groupings past the common case, bit-exact against the oracle:
    more than 1,024 tiles of 1,024 slots (the counting grouping: per-variable
    atomics, scan, fill), more than 1M variables (the tile sort with buckets of
    2,048 variables, 977 tiles: the bucket ranges read two tiles a thread), and
    391 tiles (one a thread).  Zipf-drawn rows give long segments; a twentieth
    of the slots hit no variable."""
    from engraft_ngram_amd import descent as D
    _say(f"scatter_grad grouping, {n_slots} slots over {n_var} variables")
    rng = np.random.default_rng(71)
    ids = np.sort(rng.choice(np.arange(0, 8 * n_var, 2, dtype=np.int64), size=n_var, replace=False)).astype(np.int32)
    pick = (rng.zipf(1.2, size=n_slots) - 1) % n_var
    rows = ids[pick].astype(np.int64)
    rows[rng.random(n_slots) < 0.05] += 1  # odd: no variable
    rows = rows.astype(np.int32).reshape(-1, 1)
    d = torch.from_numpy(rng.standard_normal((n_slots, 64), dtype=np.float32)).to(cuda)
    got = D.scatter_grad(d, torch.from_numpy(rows), torch.from_numpy(ids), 64).cpu().numpy()
    exp, hits = B.scatter_grad(d.cpu().numpy(), rows, ids)
    _say(f"longest segment {hits.max()}, variables hit {(hits > 0).sum()}")
    assert hits.max() > 1000
    assert np.array_equal(got, exp)


def test_descent_step_config2_full_size(cuda):
    """BASELINE config 2 at its own size: the config-1 table and batch, d_residual
    [16384, 2048] bf16 ~ N(0, 1e-3), duplicates merged deterministically, Adam
    (lr 1e-3, betas 0.9/0.999, eps 1e-8) on the touched rows, requantised to Q8_0."""
    from engraft_ngram_amd import descent as D
    _say("descent cfg2 (43.5 GB table)")
    c = CFG1
    spec = synthetic_spec(n_rows=c["n_rows"], seed=300)
    tab = G.device_table(spec, "q8_0", c["n_rows"], 128, seed=301)
    n = c["batch"] * c["seq"]
    tokens = synth.zipf_tokens(302, n, c["vocab"])
    _, rows = tab.forward(torch.from_numpy(tokens), None, seq_len=c["seq"], return_rows=True)
    rows = rows[0]
    g = torch.Generator(device=cuda).manual_seed(303)
    d_res = (torch.randn((n, 2048), generator=g, device=cuda) * 1e-3).to(torch.bfloat16)
    st = D.DescentState.from_rows(tab, rows)
    st2 = D.DescentState.from_rows(tab, rows)
    st.step(d_res, rows, lr=1e-3)
    st2.step(d_res, rows, lr=1e-3)
    torch.cuda.synchronize()
    ids = st.ids.cpu().numpy()
    rows_np = rows.cpu().numpy()
    assert np.array_equal(ids, np.unique(rows_np))
    master0 = G.synth_fetch("q8_0", 301, 128)(ids)
    grad, hits = B.scatter_grad(d_res.float().cpu().numpy(), rows_np, ids)
    _say(f"cfg2: {ids.size} unique rows, longest segment {hits.max()}")
    p1, m1, v1 = B.adam_step(master0, grad, np.zeros_like(master0), np.zeros_like(master0), 1, 1e-3)
    got = st.master.cpu().numpy()
    _rel_ok(got, p1)
    assert np.array_equal(got, p1)
    assert np.array_equal(st.m.cpu().numpy(), m1) and np.array_equal(st.v.cpu().numpy(), v1)
    q, dq = F.quant_q8_0(got)
    assert np.array_equal(st.quant.payload.cpu().numpy().view(np.int8), q)
    assert np.array_equal(st.quant.scales.cpu().numpy(), dq)
    # bitwise repeatable
    assert torch.equal(st.master, st2.master) and torch.equal(st.quant.payload, st2.quant.payload)
    del tab, st, st2
    torch.cuda.empty_cache()


def test_sparse_multistep_against_oracle(cuda):
    """Three steps on different batches: only the rows a batch hits step
    (their moments lazily), with the global step count in the bias corrections."""
    from engraft_ngram_amd import descent as D
    spec = synthetic_spec(n_rows=16 * 4000, seed=71)
    tab = G.device_table(spec, "q8_0", 16 * 4000, 128, seed=72)
    batches = [synth.zipf_tokens(73 + k, 1024, 5000) for k in range(3)]
    all_rows = [H.ngram_rows_np(spec, b) for b in batches]
    st = D.DescentState.from_rows(tab, torch.from_numpy(np.concatenate(all_rows).astype(np.int32)))
    ids = st.ids.cpu().numpy()
    p = G.synth_fetch("q8_0", 72, 128)(ids)
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    for k, r in enumerate(all_rows, start=1):
        d = (torch.randn((1024, 2048), device=cuda) * 1e-3).to(torch.bfloat16)
        st.step(d, torch.from_numpy(r.astype(np.int32)), lr=2e-3)
        grad, hits = B.scatter_grad(d.float().cpu().numpy(), r, ids)
        p, m, v = B.adam_step(p, grad, m, v, k, 2e-3, touched=hits > 0)
    got = st.master.cpu().numpy()
    _rel_ok(got, p)
    assert np.array_equal(got, p)
    assert np.array_equal(st.v.cpu().numpy(), v)


def test_dense_with_pull_term_against_torch_adam(cuda):
    """The reference's own step (engraft/descend_corpus.py:921-947): dense
    torch.optim.Adam over rows_var with the pull term mu*||rows_var-rows0||^2/
    ||rows0||^2, three steps, against torch on the CPU (1e-5 relative)."""
    from engraft_ngram_amd import descent as D
    spec = synthetic_spec(n_rows=16 * 2000, seed=81)
    tab = G.device_table(spec, "q8_0", 16 * 2000, 128, seed=82)
    tokens = synth.zipf_tokens(83, 2048, 3000)
    rows = H.ngram_rows_np(spec, tokens)
    st = D.DescentState.from_rows(tab, torch.from_numpy(rows.astype(np.int32)))
    ids = st.ids.cpu().numpy()
    rows0 = G.synth_fetch("q8_0", 82, 128)(ids)
    rv = torch.from_numpy(rows0.copy()).requires_grad_(True)
    r0 = torch.from_numpy(rows0.copy())
    opt = torch.optim.Adam([rv], lr=1e-3)
    mu = 0.1
    for k in range(3):
        # a batch that hits only part of the variables: the dense step moves the rest too
        sub = rows[k * 600:(k + 1) * 600]
        d = (torch.randn((600, 2048), device=cuda) * 1e-3).to(torch.bfloat16)
        st.step(d, torch.from_numpy(sub.astype(np.int32)), lr=1e-3, dense=True, mu=mu)
        grad, _ = B.scatter_grad(d.float().cpu().numpy(), sub, ids)
        opt.zero_grad()
        rv.grad = torch.from_numpy(grad)
        reg = mu * ((rv - r0).pow(2).sum() / r0.pow(2).sum().clamp_min(1e-12))
        reg.backward()
        opt.step()
    _rel_ok(st.master.cpu().numpy(), rv.detach().numpy())


@pytest.mark.parametrize("anchor", [True, False])
def test_warm_start_pull_term_anchor(cuda, anchor):
    """A warm start (rows_var starting away from the true rows): with
    ``anchor`` the pull term's rows0 are the warm rows, as in
    engraft/descend_corpus.py:780-781, 935-939; without it rows0 are the true
    rows of the base table, as in engraft/replica/descend.py:141, 252.  Three
    dense steps against torch.optim.Adam on the CPU with that rows0."""
    from engraft_ngram_amd import descent as D
    spec = synthetic_spec(n_rows=16 * 2000, seed=181)
    tab = G.device_table(spec, "q8_0", 16 * 2000, 128, seed=182)
    tokens = synth.zipf_tokens(183, 1024, 3000)
    rows = H.ngram_rows_np(spec, tokens)
    ids = np.unique(rows).astype(np.int32)
    true = G.synth_fetch("q8_0", 182, 128)(ids)
    warm = (true + np.random.default_rng(184).standard_normal(true.shape).astype(np.float32) * 0.01).astype(
        np.float32)
    ids_d = torch.from_numpy(ids).to(cuda)
    warm_d = torch.from_numpy(warm).to(cuda)
    st = D.DescentState(ids_d, warm_d.clone(), base=tab, anchor=warm_d.clone() if anchor else None)
    rv = torch.from_numpy(warm.copy()).requires_grad_(True)
    r0 = torch.from_numpy((warm if anchor else true).copy())
    opt = torch.optim.Adam([rv], lr=1e-3)
    mu = 0.1
    for k in range(3):
        sub = rows[k * 300:(k + 1) * 300]
        d = (torch.randn((300, 2048), device=cuda) * 1e-3).to(torch.bfloat16)
        st.step(d, torch.from_numpy(sub.astype(np.int32)), lr=1e-3, dense=True, mu=mu)
        grad, _ = B.scatter_grad(d.float().cpu().numpy(), sub, ids)
        opt.zero_grad()
        rv.grad = torch.from_numpy(grad)
        reg = mu * ((rv - r0).pow(2).sum() / r0.pow(2).sum().clamp_min(1e-12))
        reg.backward()
        opt.step()
    _rel_ok(st.master.cpu().numpy(), rv.detach().numpy())


def test_updated_rows_read_back_through_forward_overlay(cuda):
    """The requantised rows of a step are what the next forward reads
    (overlay-vs-base resolved per id on the device)."""
    from engraft_ngram_amd import descent as D
    spec = synthetic_spec(n_rows=16 * 3000, seed=91)
    tab = G.device_table(spec, "q8_0", 16 * 3000, 128, seed=92)
    tokens = synth.zipf_tokens(93, 1024, 4000)
    rows = H.ngram_rows_np(spec, tokens)
    st = D.DescentState.from_rows(tab, torch.from_numpy(rows[:500].astype(np.int32)))
    d = (torch.randn((500, 2048), device=cuda) * 1e-2).to(torch.bfloat16)
    st.step(d, torch.from_numpy(rows[:500].astype(np.int32)), lr=1e-2)
    res = G.residual(1024, 2048, seed=94)
    for quantized in (True, False):
        out = tab.forward(torch.from_numpy(tokens), res, overlay=st.overlay(quantized=quantized))
        ids = st.ids.cpu().numpy()
        if quantized:
            vals = F.dequant_q8_0(st.quant.payload.cpu().numpy().view(np.int8), st.quant.scales.cpu().numpy())
        else:
            vals = st.master.cpu().numpy()
        _, _, exp = FW.forward(spec, tokens, G.synth_fetch("q8_0", 92, 128), G.bf16_bits(res),
                               overlay=(ids, vals))
        G.assert_out_matches(G.bf16_bits(out), exp)


@pytest.mark.parametrize("fmt,dim", [("q8_0", 128), ("mxfp8", 128), ("q8_0", 160), ("mxfp8", 64)])
def test_quantised_overlay_valid_before_first_step(cuda, fmt, dim):
    """A new state's requantised rows are its master rows under the
    requantisation rule (bit-exact), so the overlay is whole before any step;
    eg_quantize_rows with destination rows writes exactly those rows."""
    import ctypes

    from engraft_ngram_amd import _lib
    from engraft_ngram_amd import descent as D
    _say(f"quantise fmt={fmt} dim={dim}")
    g = torch.Generator(device=cuda).manual_seed(101)
    n = 3000
    master = torch.randn((n, dim), generator=g, device=cuda) * 0.02
    master[7, :32] = 0.0  # an all-zero block
    ids = torch.arange(0, 3 * n, 3, dtype=torch.int32, device=cuda)
    st = D.DescentState(ids, master.clone(), quant_fmt=fmt)
    rule = F.quant_q8_0 if fmt == "q8_0" else F.quant_mxfp8
    q_exp, s_exp = rule(master.cpu().numpy())
    q_got = st.quant.payload.view(torch.uint8).cpu().numpy().reshape(n, dim)
    s_got = st.quant.scales.view(torch.uint8).cpu().numpy().reshape(n, -1)
    assert np.array_equal(q_got, q_exp.view(np.uint8))
    assert np.array_equal(s_got, np.ascontiguousarray(s_exp).view(np.uint8).reshape(n, -1))
    # scatter form: rows 5, 0 and 2999 rewritten from new values; -1 and n are skipped
    src = torch.randn((5, dim), generator=g, device=cuda) * 0.05
    dst = torch.tensor([5, -1, 0, n, n - 1], dtype=torch.int32, device=cuda)
    tab = st.quant.c_table()
    _lib.call("eg_quantize_rows", _lib.ptr(src), 5, dim, _lib.ptr(dst), ctypes.byref(tab), _lib.stream_ptr(cuda))
    q2, s2 = rule(src.cpu().numpy())
    q_now = st.quant.payload.view(torch.uint8).cpu().numpy().reshape(n, dim)
    s_now = st.quant.scales.view(torch.uint8).cpu().numpy().reshape(n, -1)
    q_ref = q_exp.view(np.uint8).copy()
    s_ref = np.ascontiguousarray(s_exp).view(np.uint8).reshape(n, -1).copy()
    for i, r in ((0, 5), (2, 0), (4, n - 1)):
        q_ref[r] = q2.view(np.uint8)[i]
        s_ref[r] = np.ascontiguousarray(s2).view(np.uint8).reshape(5, -1)[i]
    assert np.array_equal(q_now, q_ref)
    assert np.array_equal(s_now, s_ref)


def test_frozen_rows_masked_step_against_torch_adam(cuda):
    """The masked step (engraft/replica/descend.py:262-271): dense Adam with the
    pull term, the frozen rows' gradient zeroed after the pull's backward, the
    frozen rows restored to rows0 after the step -- against torch on the CPU.
    The mask is off for the first step, so a frozen row carries moments."""
    from engraft_ngram_amd import descent as D
    spec = synthetic_spec(n_rows=16 * 2000, seed=111)
    tab = G.device_table(spec, "q8_0", 16 * 2000, 128, seed=112)
    tokens = synth.zipf_tokens(113, 2048, 3000)
    rows = H.ngram_rows_np(spec, tokens)
    st = D.DescentState.from_rows(tab, torch.from_numpy(rows.astype(np.int32)))
    ids = st.ids.cpu().numpy()
    rows0 = G.synth_fetch("q8_0", 112, 128)(ids)
    rv = torch.from_numpy(rows0.copy()).requires_grad_(True)
    r0 = torch.from_numpy(rows0.copy())
    opt = torch.optim.Adam([rv], lr=1e-3)
    mu = 0.1
    rng = np.random.default_rng(114)
    row_mask = rng.random(ids.size) < 0.5  # True: the row moves
    frozen_t = torch.from_numpy(~row_mask)
    for k in range(3):
        sub = rows[k * 600:(k + 1) * 600]
        d = (torch.randn((600, 2048), device=cuda) * 1e-3).to(torch.bfloat16)
        masked = k > 0
        st.step(d, torch.from_numpy(sub.astype(np.int32)), lr=1e-3, dense=True, mu=mu,
                frozen=~row_mask if masked else None)
        grad, _ = B.scatter_grad(d.float().cpu().numpy(), sub, ids)
        opt.zero_grad()
        rv.grad = torch.from_numpy(grad)
        reg = mu * ((rv - r0).pow(2).sum() / r0.pow(2).sum().clamp_min(1e-12))
        reg.backward()
        if masked:
            rv.grad[frozen_t] = 0.0
        opt.step()
        if masked:
            with torch.no_grad():
                rv[frozen_t] = r0[frozen_t]
    got = st.master.cpu().numpy()
    exp = rv.detach().numpy()
    _rel_ok(got, exp)
    assert np.array_equal(got[~row_mask], rows0[~row_mask])
    state = opt.state[rv]
    _rel_ok(st.m.cpu().numpy(), state["exp_avg"].numpy(), tol=1e-4)
    # the frozen rows' requantised copy is the rule applied to rows0
    q_exp, s_exp = F.quant_q8_0(rows0[~row_mask])
    fz = np.nonzero(~row_mask)[0]
    assert np.array_equal(st.quant.payload.cpu().numpy().view(np.int8)[fz], q_exp)
    assert np.array_equal(st.quant.scales.cpu().numpy().view(np.float16)[fz], s_exp)


def test_descent_step_edge_cases(cuda):
    """A step without slots (sparse: nothing moves; dense: the zero-gradient step,
    whose pull term is zero at the start rows, leaves the rows as they are), and
    slots that hit no variable."""
    from engraft_ngram_amd import descent as D
    _say("descent edge cases")
    spec = synthetic_spec(n_rows=16 * 1000, seed=101)
    tab = G.device_table(spec, "q8_0", 16 * 1000, 128, seed=102)
    tokens = synth.zipf_tokens(103, 256, 2000)
    rows = H.ngram_rows_np(spec, tokens).astype(np.int32)
    st = D.DescentState.from_rows(tab, torch.from_numpy(rows))
    p0, q0 = st.master.clone(), st.quant.payload.clone()
    none_d = torch.zeros((0, 16 * 128), dtype=torch.bfloat16, device=cuda)
    none_r = torch.zeros((0, 16), dtype=torch.int32)
    st.step(none_d, none_r, lr=1e-3)
    assert st.step_count == 1 and torch.equal(st.master, p0) and torch.equal(st.quant.payload, q0)
    st.step(none_d, none_r, lr=1e-3, dense=True, mu=0.1)
    assert st.step_count == 2 and torch.equal(st.master, p0) and float(st.m.abs().max()) == 0.0
    # slots whose rows are not variables
    ids = st.ids.cpu().numpy()
    free = int(np.setdiff1d(np.arange(16 * 1000), ids)[0])
    d = (torch.randn((256, 16 * 128), device=cuda) * 1e-3).to(torch.bfloat16)
    st.step(d, torch.full((256, 16), free, dtype=torch.int32), lr=1e-3)
    assert torch.equal(st.master, p0)


def _index_group(row: int, bits: int) -> int:
    """The row index's hash group of a row (Fibonacci hashing, groups of 8)."""
    return (((row * 0x9E3779B1) & 0xFFFFFFFF) >> (32 - bits)) >> 3


@pytest.mark.parametrize("cap,n_ids", [(8, 4), (16, 8)])
def test_row_index_small_and_full_groups(cuda, cap, n_ids):
    """The row index probes aligned groups of 8 entries.  A table of 8 entries
    (one group), and a table of 16 whose first group is full (every id hashes
    into it; lookups of absent rows of that group go on to the second), give
    the same step, bit for bit, as the state's own index."""
    from engraft_ngram_amd import _lib
    from engraft_ngram_amd import descent as D
    _say(f"row index of {cap} entries, {n_ids} ids")
    bits = cap.bit_length() - 1
    grp0 = [r for r in range(1, 200000) if _index_group(r, bits) == 0]
    ids = np.array(sorted(grp0[:n_ids]), dtype=np.int32)
    absent = grp0[n_ids:n_ids + 8] + [r for r in range(1, 200000) if _index_group(r, bits) != 0][:8]
    rng = np.random.default_rng(7)
    rows = rng.choice(np.concatenate([ids, np.array(absent, dtype=np.int32)]), size=(64, 4)).astype(np.int32)
    rows.reshape(-1)[:n_ids] = ids  # every id is some slot's row
    g = torch.Generator(device=cuda).manual_seed(8)
    master = torch.randn((n_ids, 128), generator=g, device=cuda) * 0.02
    d = (torch.randn((64, 4 * 128), generator=g, device=cuda) * 1e-3).to(torch.bfloat16)
    ref = D.DescentState(torch.from_numpy(ids).to(cuda), master.clone())
    small = D.DescentState(torch.from_numpy(ids).to(cuda), master.clone())
    small.index = torch.empty(cap, dtype=torch.int64, device=cuda)
    _lib.call("eg_build_row_index", _lib.ptr(small.ids), n_ids, _lib.ptr(small.index), cap, _lib.stream_ptr(cuda))
    table = small.index.cpu().numpy()
    assert (table[:8] != -1).sum() == min(n_ids, 8)  # every id sits in the first group
    r = torch.from_numpy(rows).to(cuda)
    for st in (ref, small):
        st.step(d, r, lr=1e-3)
        st.step(d, r, lr=1e-3)
    torch.cuda.synchronize()
    for a, b in ((ref.master, small.master), (ref.m, small.m), (ref.v, small.v),
                 (ref.quant.payload, small.quant.payload), (ref.quant.scales, small.quant.scales)):
        assert torch.equal(a, b)
    assert not torch.equal(ref.master, master)  # the step moved the rows


def test_planned_steps_on_a_second_stream(cuda):
    """A descent loop that groups the next batch's slots on a second stream
    while the current step runs (DescentState.plan + step(plan=...), i.e.
    eg_descent_plan + eg_descent_apply, two plan buffers alternating): every
    step bitwise the step that groups its own slots, over batches whose rows
    differ, and the plan's misuse refused."""
    from engraft_ngram_amd import descent as D
    _say("planned descent steps on a second stream")
    spec = synthetic_spec(n_rows=16 * 4000, seed=81)
    tab = G.device_table(spec, "q8_0", 16 * 4000, 128, seed=82)
    batches = [synth.zipf_tokens(83 + k, 1024, 5000) for k in range(5)]
    all_rows = [torch.from_numpy(H.ngram_rows_np(spec, b).astype(np.int32)).to(cuda) for b in batches]
    union = torch.cat(all_rows)
    ref = D.DescentState.from_rows(tab, union)
    st = D.DescentState.from_rows(tab, union)
    g = torch.Generator(device=cuda).manual_seed(84)
    d_res = [(torch.randn((1024, 2048), generator=g, device=cuda) * 1e-3).to(torch.bfloat16) for _ in batches]
    for d, r in zip(d_res, all_rows):
        ref.step(d, r, lr=2e-3)
    main = torch.cuda.current_stream(cuda)
    side = torch.cuda.Stream(cuda)  # default priority
    side.wait_stream(main)  # the row ids were made on the main stream
    plans = [None, None]
    planned = [torch.cuda.Event(), torch.cuda.Event()]
    applied = [torch.cuda.Event(), torch.cuda.Event()]
    plans[0] = st.plan(all_rows[0])
    planned[0].record(main)
    for i in range(len(batches)):
        if i + 1 < len(batches):
            j = (i + 1) % 2
            with torch.cuda.stream(side):
                if plans[j] is not None:
                    side.wait_event(applied[j])  # the buffer's previous step has read it
                plans[j] = st.plan(all_rows[i + 1], plan=plans[j])
                planned[j].record(side)
        main.wait_event(planned[i % 2])
        st.step(d_res[i], plan=plans[i % 2], lr=2e-3)
        applied[i % 2].record(main)
    torch.cuda.synchronize()
    assert st.step_count == ref.step_count == len(batches)
    assert torch.equal(st.master, ref.master) and torch.equal(st.m, ref.m) and torch.equal(st.v, ref.v)
    assert torch.equal(st.quant.payload, ref.quant.payload) and torch.equal(st.quant.scales, ref.quant.scales)
    other = D.DescentState.from_rows(tab, union)
    p = other.plan(all_rows[0])
    with pytest.raises(ValueError):
        st.step(d_res[0], plan=p, lr=2e-3)
    with pytest.raises(ValueError):
        other.step(d_res[0], all_rows[0][:512], plan=p, lr=2e-3)
    with pytest.raises(ValueError):
        other.step(d_res[0], plan=p, lr=2e-3, no_alloc=True)


def test_descent_from_the_forwards_slot_variables(cuda):
    """The forward over the state's overlay writes each slot's variable
    (eg_forward_slots: the rank of its row among the ids, -1 for base rows,
    as the oracle's binary search finds it); the step grouped from those
    (eg_descent_plan_slots, no row lookup) is bitwise the step from the rows,
    including slots that hit no variable."""
    from engraft_ngram_amd import descent as D
    from engraft_ngram_amd import table as T
    _say("descent from the forward's slot variables")
    spec = synthetic_spec(n_rows=16 * 4000, seed=91)
    tab = G.device_table(spec, "q8_0", 16 * 4000, 128, seed=92)
    tokens = synth.zipf_tokens(93, 4096, 5000)
    rows_np = H.ngram_rows_np(spec, tokens, seq_len=1024).astype(np.int32)
    # variables: the rows of the first half of the batch only, so the second half has misses
    st = D.DescentState.from_rows(tab, torch.from_numpy(rows_np[:2048]))
    ref = D.DescentState.from_rows(tab, torch.from_numpy(rows_np[:2048]))
    ids = st.ids.cpu().numpy()
    res = G.residual(tokens.size, 2048, seed=94)
    call = T.PreparedForward([tab], torch.from_numpy(tokens), res, overlays=[st.overlay()], seq_len=1024,
                             return_rows=True, return_slot_vars=True)
    call()
    torch.cuda.synchronize()
    sv = call.slot_vars[0].cpu().numpy()
    assert np.array_equal(call.rows[0].cpu().numpy(), rows_np)
    pos = np.searchsorted(ids, rows_np)
    hit = (pos < ids.size) & (ids[np.minimum(pos, ids.size - 1)] == rows_np)
    exp = np.where(hit, pos, -1)
    assert np.array_equal(sv, exp) and (sv == -1).any() and (sv >= 0).any()
    g = torch.Generator(device=cuda).manual_seed(95)
    for k in range(2):
        d = (torch.randn((4096, 2048), generator=g, device=cuda) * 1e-3).to(torch.bfloat16)
        st.step(d, slot_var=call.slot_vars[0], lr=1e-3)
        ref.step(d, torch.from_numpy(rows_np), lr=1e-3)
    torch.cuda.synchronize()
    assert torch.equal(st.master, ref.master) and torch.equal(st.m, ref.m) and torch.equal(st.v, ref.v)
    assert torch.equal(st.quant.payload, ref.quant.payload) and torch.equal(st.quant.scales, ref.quant.scales)
    with pytest.raises(ValueError):
        st.step(d, torch.from_numpy(rows_np), slot_var=call.slot_vars[0], lr=1e-3)
