"""Helpers for the GPU parity tests: build device tables from oracle specs and
copy device tensors back as numpy bit patterns."""
from __future__ import annotations

import numpy as np
import torch

from engraft_ngram_amd import table as T
from oracle import formats as F
from oracle import forward as FW
from oracle import synth
from oracle.hash import HashSpec


def device_table(spec: HashSpec, fmt: str, n_rows: int, dim: int, seed: int, sigma: float = 0.02,
                 device="cuda:0") -> T.DeviceTable:
    return T.DeviceTable.synthetic(
        fmt, n_rows, dim, seed=seed, sigma=sigma, eos_token_id=spec.eos_token_id, ngram_size=spec.ngram_size,
        heads_per_ngram=spec.heads_per_ngram, layer_multipliers=spec.layer_multipliers,
        head_vocab_sizes=spec.head_vocab_sizes, head_offsets=spec.head_offsets,
        head_multipliers=spec.head_multipliers, device=device)


def table_from_arrays(spec: HashSpec, fmt: str, dim: int, payload: np.ndarray, scales=None,
                      device="cuda:0") -> T.DeviceTable:
    n = payload.shape[0]
    shp, dt = T.payload_shape(fmt, n, dim)
    p = torch.from_numpy(np.ascontiguousarray(payload)).view(dt).reshape(shp).to(device)
    s = None
    ss = T.scales_shape(fmt, n, dim)
    if ss is not None:
        s = torch.from_numpy(np.ascontiguousarray(scales)).view(ss[1]).reshape(ss[0]).to(device)
    store = T.RowStore(fmt, dim, p, s)
    return T.DeviceTable(store, eos_token_id=spec.eos_token_id, ngram_size=spec.ngram_size,
                         heads_per_ngram=spec.heads_per_ngram, layer_multipliers=spec.layer_multipliers,
                         head_vocab_sizes=spec.head_vocab_sizes, head_offsets=spec.head_offsets,
                         head_multipliers=spec.head_multipliers)


def synth_fetch(fmt: str, seed: int, dim: int, sigma: float = 0.02):
    """Oracle row fetcher that regenerates rows of the seeded synthetic table."""
    def fetch(ids):
        ids = np.asarray(ids, dtype=np.int64)
        uniq, inv = np.unique(ids, return_inverse=True)
        return synth.synth_dequant(fmt, seed, uniq, dim, sigma)[inv.reshape(-1)]
    return fetch


def bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def residual(n: int, w: int, seed: int, device="cuda:0") -> torch.Tensor:
    g = torch.Generator(device=device).manual_seed(seed)
    return torch.randn((n, w), generator=g, device=device, dtype=torch.float32).to(torch.bfloat16)


def assert_out_matches(out_bits: np.ndarray, exp_bits: np.ndarray) -> None:
    """Bit-exact, and (the stated bar) within 1e-3 relative of the oracle."""
    got = F.bf16_bits_to_f32(out_bits).astype(np.float64)
    exp = F.bf16_bits_to_f32(exp_bits).astype(np.float64)
    rel = np.abs(got - exp) / np.maximum(np.abs(exp), 1e-30)
    assert np.all((rel <= 1e-3) | (got == exp)), f"max rel err {rel.max()}"
    n_diff = int((out_bits != exp_bits).sum())
    assert n_diff == 0, f"{n_diff} bf16 outputs differ from the oracle"


__all__ = ["device_table", "table_from_arrays", "synth_fetch", "bf16_bits", "residual", "assert_out_matches",
           "FW", "F", "synth"]


def f32_table(spec: HashSpec, dim: int, seed: int, device="cuda:0"):
    """A small F32 device table of normal rows (x0.05) and its oracle fetch."""
    n = int(sum(spec.head_vocab_sizes))
    data = (np.random.default_rng(seed).standard_normal((n, dim)) * 0.05).astype(np.float32)
    return table_from_arrays(spec, "f32", dim, data, device=device), (lambda ids: data[np.asarray(ids, np.int64)])
