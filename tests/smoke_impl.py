"""``__graft_entry__.smoke()``: one small invocation of the table path on
cuda:0, checked against the CPU oracle."""
from __future__ import annotations

import numpy as np
import torch

from oracle import forward as FW
from oracle import synth
from tests import gpu_util as G
from tests.params import synthetic_spec


def run() -> None:
    assert torch.cuda.is_available(), "smoke() needs a GPU"
    spec = synthetic_spec(n_rows=16 * 8192, seed=1)
    tab = G.device_table(spec, "q8_0", 16 * 8192, 128, seed=2)
    tokens = synth.zipf_tokens(3, 2 * 512, 151_936)
    res = G.residual(tokens.size, 2048, seed=4)
    out, rows = tab.forward(torch.from_numpy(tokens), res, seq_len=512, return_rows=True)
    exp_rows, _, exp_out = FW.forward(spec, tokens, G.synth_fetch("q8_0", 2, 128), G.bf16_bits(res),
                                      seq_len=512)
    assert np.array_equal(rows[0].cpu().numpy(), exp_rows), "row ids differ from the oracle"
    G.assert_out_matches(G.bf16_bits(out), exp_out)
    print("smoke: forward (hash -> gather -> dequant -> residual add) matches the oracle", flush=True)

    # one descent step on the rows just read: deterministic scatter + Adam + requant
    from engraft_ngram_amd import descent as D
    from oracle import backward as B

    d = (torch.randn((tokens.size, 2048), generator=torch.Generator(device="cuda").manual_seed(5), device="cuda")
         * 1e-3).to(torch.bfloat16)
    st = D.DescentState.from_rows(tab, rows[0])
    st.step(d, rows[0], lr=1e-3)
    ids = st.ids.cpu().numpy()
    grad, _ = B.scatter_grad(d.float().cpu().numpy(), exp_rows, ids)
    p0 = G.synth_fetch("q8_0", 2, 128)(ids)
    p1, _, _ = B.adam_step(p0, grad, np.zeros_like(p0), np.zeros_like(p0), 1, 1e-3)
    assert np.array_equal(st.master.cpu().numpy(), p1), "descent step differs from the oracle"
    print("smoke: descent step (scatter + Adam) matches the oracle", flush=True)
