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
