"""The descent loop end to end on the device, as the reference's
tests/test_seq.py:48-88 runs it on the CPU: a packed two-fragment sequence
(segment ids [0,0,0,0,0,1,1,1]), overlay rows as variables, the PLE block as
the consumer, five Adam steps with a decreasing loss, then a .pleo round trip.

Two device loops against one CPU oracle loop:
  A  OverlayEmb (differentiable gather) -> ple_forward -> loss -> torch Adam
  B  eg_forward with the state's fp32 rows as overlay -> ple_forward -> loss ->
     DescentState.step (eg_descent_step, the reference's dense Adam)
Oracle: oracle.overlay_emb.build -> oracle.ple.ple_forward (torch fp32, CPU)
-> autograd to emb -> the oracle's slot-ordered scatter -> torch.optim.Adam.

Bar: losses within 1e-4 relative of the oracle's at every step, the rows after
five steps within 1e-4 of the largest entry; the .pleo round trip bit-exact."""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import backward as B
from oracle import overlay_emb as OE
from oracle import ple as P
from tests import gpu_util as G
from tests.params import fake_table_spec
from tests.test_oracle_ple import ple_weights

pytestmark = pytest.mark.gpu


class _HP:
    hc_mult = 4
    n_embd = 2560
    f_norm_rms_eps = 1e-6
    ple_ngram_size = 3


def test_packed_overlay_descent_through_ple(cuda, tmp_path):
    from engraft_ngram_amd import lens, ple
    from engraft_ngram_amd.descent import DescentState
    from engraft_ngram_amd.pack import pack_fragments, seg_starts_from_segment_ids
    from engraft_ngram_amd.seq import OverlayEmb
    print("[gpu-test] descent loop through ple_forward", file=sys.stderr, flush=True)
    spec = fake_table_spec(7)
    tab, fetch = G.f32_table(spec, 160, seed=8)
    packed = pack_fragments([[3, 5, 7, 2], [9, 4, 6]], spec.eos_token_id, max_len=64)[0]
    assert packed.segment_ids.tolist() == [0, 0, 0, 0, 0, 1, 1, 1]
    tokens = packed.tokens
    n = len(tokens) - 1  # prefix positions (the last token is only a target)
    seg = packed.segment_ids.numpy()
    rows, *_ = OE.build_plan(spec, tokens, {}, n, 0, seg)
    ids = sorted({int(rows[0, 0]), int(rows[5, 9]), int(rows[6, 3])})
    row_map = {g: i for i, g in enumerate(ids)}
    keys = OE.slot_keys(*OE.build_plan(spec, tokens, row_map, n, 0, seg)[2:5], n, 16)
    rows0 = fetch(np.array(ids))
    hc, d = 4, 2560
    w = ple_weights(hc, d, seed=9)
    g = torch.Generator().manual_seed(10)
    hidden = torch.randn((n, hc, d), generator=g) * 0.1
    target = torch.randn((n, hc, d), generator=g) * 0.1
    lr, steps = 0.01, 5

    # oracle loop (CPU)
    rv_c = torch.from_numpy(rows0.copy()).requires_grad_(True)
    opt_c = torch.optim.Adam([rv_c], lr=lr)
    loss_c = []
    for _ in range(steps):
        emb_np, *_ = OE.build(spec, tokens, row_map, rv_c.detach().numpy(), n, fetch, segment_ids=seg)
        emb = torch.from_numpy(emb_np).requires_grad_(True)
        out, _, _, _ = P.ple_forward(emb, hidden, w, torch.zeros(0, hc, d), hc, d, 1e-6, 3)
        loss = ((out - target) ** 2).mean()
        loss.backward()
        grad, _ = B.scatter_grad_keys(emb.grad.numpy(), keys, 16, len(ids))
        opt_c.zero_grad()
        rv_c.grad = torch.from_numpy(grad)
        opt_c.step()
        loss_c.append(float(loss.detach()))
    assert loss_c[-1] < loss_c[0]

    wd = ple.PleWeights(**{k: v.to(cuda) for k, v in w.items()})
    hd, td = hidden.to(cuda), target.to(cuda)
    h0 = torch.zeros(0, hc, d, device=cuda)

    # loop A: OverlayEmb + torch Adam on the device
    rv = torch.from_numpy(rows0.copy()).to(cuda).requires_grad_(True)
    opt = torch.optim.Adam([rv], lr=lr)
    loss_a = []
    for _ in range(steps):
        opt.zero_grad()
        emb = OverlayEmb(tab, tokens, rv, row_map, segment_ids=packed.segment_ids).build(n)
        out, _ = ple.ple_forward(emb, hd, wd, h0, _HP)
        loss = ((out - td) ** 2).mean()
        loss.backward()
        opt.step()
        loss_a.append(float(loss.detach()))

    # loop B: the fused forward with the state's rows + eg_descent_step
    st = DescentState(torch.tensor(ids, dtype=torch.int32, device=cuda),
                      torch.from_numpy(rows0.copy()).to(cuda), quant_fmt=None, base=tab)
    tok = torch.from_numpy(np.asarray(tokens[:n], dtype=np.int64)).to(cuda)
    seg_start = seg_starts_from_segment_ids(packed.segment_ids)
    slot_rows = tab.rows(tok, seg_start=seg_start)
    loss_b = []
    for _ in range(steps):
        emb = tab.forward(tok, None, overlay=st.overlay(quantized=False), seg_start=seg_start)
        emb.requires_grad_(True)
        out, _ = ple.ple_forward(emb, hd, wd, h0, _HP)
        loss = ((out - td) ** 2).mean()
        (d_emb,) = torch.autograd.grad(loss, emb)
        st.step(d_emb.contiguous(), slot_rows, lr=lr, dense=True)
        loss_b.append(float(loss.detach()))

    for got in (loss_a, loss_b):
        np.testing.assert_allclose(got, loss_c, rtol=1e-4)
    scale = float(rv_c.detach().abs().max())
    for got in (rv.detach(), st.master):
        assert float((got.cpu() - rv_c.detach()).abs().max()) <= 1e-4 * scale

    path = tmp_path / "smoke.pleo"
    data = st.master.cpu().numpy()
    lens.write_pleo(path, np.array(ids, dtype=np.int32), data)
    r_read, d_read = lens.read_pleo(path)
    assert r_read.tolist() == ids and np.array_equal(d_read, data)
