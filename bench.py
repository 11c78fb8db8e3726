#!/usr/bin/env python3
"""Benchmark of the Engram/PLE table path on one MI355X (BASELINE.json metric).

Workload: hash of the last 2 and 3 tokens into 16 row ids
per position, gather + Q8_0 dequantisation of the rows from a 320,000,000-row
table (43.5 GB in HBM), add into a bf16 residual [16384, 2048] (fp32
accumulate).  One step = one fused launch over the batch (8 x 2048 Zipf(1.1)
tokens).  Inputs are seeded synthetic data generated on the device before the
timed region.  Every step is a new batch: 16 token batches and four
residual/output sets (1.07 GB) rotate, so neither the rows a batch touches nor
its residual is served from the 256 MB Infinity Cache by a repeat of an
earlier step (repeating one batch runs ≈ 10 % faster for that reason).  The
other legs rotate their inputs the same way.

Prints ONE JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import itertools
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

METRIC = "table rows gathered/sec + achieved HBM GB/s (fwd read, bwd scatter), 320M-row table"
HBM_PEAK_GBS = 8000.0

N_ROWS, DIM, BATCH, SEQ, VOCAB, WIDTH, SLOTS = 320_000_000, 128, 8, 2048, 151_936, 2048, 16
TABLE_SEED, HASH_SEED, TOKEN_SEED, RES_SEED = 201, 200, 202, 203
TOKEN_SETS, RES_SETS = 16, 4  # token batches and residual sets rotated in the timed loop
DECODE_SEED, C4_SEED, PLE_SEED, REAL_SEED, SCAN_SEED = 300, 400, 500, 600, 700
Q8_ROW_BYTES = DIM + 2 * DIM // 32  # 128 B int8 + 4 fp16 scales = 136 B


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def forward_bytes(positions: int) -> int:
    """Algorithmic HBM bytes of one forward step: per position 16 rows x 136 B,
    residual read + output write (2 x 2 x 2048 B) and the 8-byte token."""
    return positions * (SLOTS * Q8_ROW_BYTES + 2 * 2 * WIDTH + 8)


def _hip():
    """The HIP runtime torch has loaded (same soname, so the same instance)."""
    import ctypes

    return ctypes.CDLL("libamdhip64.so.7")


class _Events:
    """hipEvent_t handles of the HIP runtime torch uses."""

    def __init__(self, n: int):
        import ctypes

        self._ct = ctypes
        self._hip = _hip()
        self._ev = []
        for _ in range(n):
            e = ctypes.c_void_p()
            if self._hip.hipEventCreate(ctypes.byref(e)) != 0:
                raise RuntimeError("hipEventCreate failed")
            self._ev.append(e)

    def __getitem__(self, i: int) -> int:
        return self._ev[i].value

    def elapsed_ms(self, a: int, b: int) -> float:
        ms = self._ct.c_float()
        if self._hip.hipEventElapsedTime(self._ct.byref(ms), self._ev[a], self._ev[b]) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def destroy(self) -> None:
        for e in self._ev:
            self._hip.hipEventDestroy(e)
        self._ev = []


def traffic_from_profile(kernel_key: str):
    """HBM bytes per launch of a kernel from the committed rocprofv3 PMC summary
    (``profiles/hbm_traffic_forward_descent_kernels_cfg1-4.md``: FETCH_SIZE x its copy-kernel factor +
    WRITE_SIZE x its factor), or None when the summary is absent."""
    path = ROOT / "profiles" / "hbm_traffic_forward_descent_kernels_cfg1-4.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith(f"traffic_bytes_per_launch {kernel_key} "):
            return int(line.split()[2])
    return None


def ramp(fn, seconds: float = 0.3, min_calls: int = 20) -> int:
    """Untimed launches of ``fn`` for at least ``seconds`` of wall time and
    ``min_calls`` calls, so that the shader clock has ramped up before a leg is
    timed whatever ``--warmup`` says; returns the number of calls."""
    import torch

    t0 = time.perf_counter()
    k = 0
    while k < min_calls or time.perf_counter() - t0 < seconds:
        fn()
        k += 1
        if k % 64 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return k


def copy_ceiling_us(n_bytes_moved: int, dev) -> float:
    """Time of the library's own streaming copy (``eg_stream_copy``: 16-byte
    non-temporal loads and stores) that reads and writes ``n_bytes_moved``
    bytes in total, warmed up, four buffer pairs rotated (so no repeat is
    served from the Infinity Cache): the practical ceiling for a kernel that
    moves that many bytes of HBM traffic."""
    import torch

    from engraft_ngram_amd import table as T

    n = max(16, (n_bytes_moved // 2) // 16 * 16)  # bytes per buffer: half read, half written
    sets = 4 if n < (256 << 20) else 1
    src = [torch.ones(n // 4, dtype=torch.int32, device=dev) for _ in range(sets)]
    dst = [torch.empty_like(src[0]) for _ in range(sets)]
    ramp(lambda: [T.stream_copy(src[i], dst[i]) for i in range(sets)], 0.2)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    best = float("inf")
    for _ in range(5):
        torch.cuda.synchronize()
        a.record()
        for i in range(40):
            T.stream_copy(src[i % sets], dst[i % sets])
        b.record()
        torch.cuda.synchronize()
        best = min(best, a.elapsed_time(b) / 40 * 1e3)
    return best


def stream_ceilings(dev) -> dict:
    """The streaming copy's rate at the residual stream alone (134.2 MB), at the
    forward's HBM traffic (198.4 MB) and at 1 GiB: the ceilings the forward is
    read against."""
    out = {}
    for name, nb in (("residual_stream_134MB", 2 * 67_108_864), ("forward_traffic_198MB", 198_385_667),
                     ("copy_1GiB", 2 * 536_870_912)):
        us = copy_ceiling_us(nb, dev)
        out[name] = {"bytes_moved": nb, "us": us, "tb_per_s": nb / (us * 1e-6) / 1e12}
    return out


def oracle_spec(hp: dict):
    from oracle import hash as OH
    return OH.HashSpec(eos_token_id=hp["eos_token_id"], ngram_size=hp["ngram_size"],
                       heads_per_ngram=hp["heads_per_ngram"], layer_multipliers=tuple(hp["layer_multipliers"]),
                       head_vocab_sizes=tuple(hp["head_vocab_sizes"]), head_offsets=tuple(hp["head_offsets"]),
                       head_multipliers=tuple(tuple(r) for r in hp["head_multipliers"]))


def log_cpu_leg(name: str, leg: dict) -> None:
    cb = leg.get("cpu_baseline")
    if cb:
        log(f"{name} cpu baseline: {cb['value']:.3g} {cb['unit']} on {cb['cores']} thread(s)")


def host_cpu() -> dict:
    """The host the CPU legs ran on: CPU model, logical CPUs, CPUs this process may use."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"model": model, "logical_cpus": os.cpu_count(), "usable_cpus": len(os.sched_getaffinity(0))}


def repeat_for(fn, budget_s: float) -> tuple[int, float]:
    """Calls fn until budget_s has passed (at least once): (calls, seconds)."""
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            return n, el


def cpu_baseline(hp: dict, tokens_np, residual_cpu, budget_s: float) -> dict:
    """The oracle's vectorized CPU restatement on the same inputs (rank 0, N=1),
    and the reference's per-position loop on the first 256 positions."""
    import numpy as np
    import torch

    from oracle import cpu_baseline as CB
    from oracle import hash as OH

    spec = oracle_spec(hp)
    t0 = time.perf_counter()
    host = CB.HostTable(N_ROWS, DIM)
    rows = OH.ngram_rows_np(spec, tokens_np, seq_len=SEQ)
    n_unique = host.populate(TABLE_SEED, rows)
    log(f"cpu baseline: host table populated ({n_unique} touched rows) in {time.perf_counter() - t0:.1f} s")
    threads = torch.get_num_threads()
    n = 0
    out = None
    t0 = time.perf_counter()
    while True:
        _, out = CB.forward_q8(spec, tokens_np, SEQ, host, residual_cpu)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    rows_per_s = n * tokens_np.size * SLOTS / el
    # the reference's loop as written: position by position, each re-hashing its prefix
    n_lit = 256
    res_bits = residual_cpu[:n_lit].view(torch.int16).numpy().view(np.uint16)
    t1 = time.perf_counter()
    lit = CB.forward_q8_literal(spec, tokens_np, n_lit, host, res_bits)
    el_lit = time.perf_counter() - t1
    literal = {"value": n_lit * SLOTS / el_lit, "unit": "rows/s", "cores": 1, "kind": "port",
               "sample": f"the first {n_lit} positions of sequence 0 in {el_lit:.2f} s: per position the scalar "
                         "hash of its whole prefix (RowSet.from_position's O(T^2) re-hash), one row read + Q8_0 "
                         "dequant per head, fp32 add -> bf16; pure Python/numpy",
               "matches_vectorized": bool(np.array_equal(lit, out[:n_lit].view(torch.int16).numpy().view(np.uint16)))}
    literal_cfg0 = cpu_literal_config0(n_lit)
    return {"result": out, "literal": literal, "literal_config0": literal_cfg0, "host": host_cpu(),
            "value": rows_per_s, "unit": "rows/s",
            "cores": threads, "kind": "port",
            "sample": (f"full config-1 step ({tokens_np.size} positions, {tokens_np.size * SLOTS} row reads) "
                       f"repeated {n}x in {el:.1f} s: numpy-uint64 hash + torch.index_select gather from a "
                       f"host table of the full 320M-row shape (touched rows materialised) + Q8_0 dequant + "
                       f"fp32 add -> bf16, {threads} torch threads"),
            "gb_per_s": n * forward_bytes(tokens_np.size) / el / 1e9, "steps": n, "seconds": el}


def cpu_literal_config0(n_pos: int) -> dict:
    """The reference's per-position loop on BASELINE config 0 (its CPU-runnable
    case: 4,194,304 bf16 rows, uniform tokens over 151,936, 16 slots, residual
    width 2048), first n_pos positions; the touched rows are generated before
    the timed loop and read one at a time inside it."""
    import numpy as np

    from engraft_ngram_amd import synthetic as S
    from oracle import cpu_baseline as CB
    from oracle import hash as OH
    from oracle import synth

    n_rows, dim, seed = 4_194_304, 128, 11
    spec = oracle_spec(S.hash_params(n_rows, seed))
    tokens = np.random.default_rng(seed + 1).integers(0, VOCAB, size=n_pos)
    rows = OH.ngram_rows_np(spec, tokens)
    uniq = np.unique(rows)
    vals = synth.synth_dequant("bf16", seed + 2, uniq, dim, 0.02)
    store = dict(zip(uniq.tolist(), vals))
    res_bits = np.random.default_rng(seed + 3).integers(0, 1 << 16, size=(n_pos, 16 * dim)).astype(np.uint16)
    res_bits &= 0x7F7F  # finite bf16 values
    t0 = time.perf_counter()
    CB.forward_literal(spec, tokens, n_pos, store.__getitem__, dim, res_bits)
    el = time.perf_counter() - t0
    return {"value": n_pos * 16 / el, "unit": "rows/s", "cores": 1, "kind": "port",
            "sample": f"BASELINE config 0 (4,194,304 bf16 rows, uniform tokens), the first {n_pos} positions in "
                      f"{el:.2f} s: per position the scalar re-hash of its prefix, a row read + dequant per head, "
                      "fp32 add -> bf16; pure Python/numpy"}


def forward_table_rows(n_rows: int, dev) -> dict:
    """The config-1 forward over a table of ``n_rows`` rows (the row ids spread
    over the whole table as at 320M rows): 16 token batches and four residual
    sets rotated, 400 launches timed after a warm-up, best of four rounds."""
    import itertools

    import torch

    from engraft_ngram_amd import synthetic as S
    from engraft_ngram_amd import table as T

    n_pos = BATCH * SEQ
    hp = S.hash_params(n_rows, HASH_SEED)
    tab = T.DeviceTable.synthetic("q8_0", n_rows, DIM, seed=TABLE_SEED, sigma=0.02, device=dev, **hp)
    toks = [torch.from_numpy(S.zipf_tokens(TOKEN_SEED + 1000 * j, n_pos, VOCAB)).to(dev) for j in range(TOKEN_SETS)]
    res = [S.residual(n_pos, WIDTH, seed=RES_SEED + i, device=dev) for i in range(RES_SETS)]
    outs = [torch.empty_like(r) for r in res]
    n_sets = max(TOKEN_SETS, RES_SETS)
    calls = [T.PreparedForward([tab], toks[i % TOKEN_SETS], res[i % RES_SETS], out=outs[i % RES_SETS], seq_len=SEQ)
             for i in range(n_sets)]
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    best = float("inf")
    for _ in range(4):
        rot = itertools.count()
        ramp(lambda: calls[next(rot) % n_sets](), 0.2)
        torch.cuda.synchronize()
        a.record()
        for i in range(400):
            calls[i % n_sets]()
        b.record()
        torch.cuda.synchronize()
        best = min(best, a.elapsed_time(b) / 400 * 1e3)
    return {"table_rows": n_rows, "table_bytes": n_rows * Q8_ROW_BYTES, "us_per_launch": best,
            "frac_of_hbm_peak": forward_bytes(n_pos) / (best * 1e-6) / (HBM_PEAK_GBS * 1e9)}


def backward_bytes(positions: int, n_unique: int) -> int:
    """Algorithmic HBM bytes of one descent step (fp32 master
    kept): d_residual read (2 B x W per position), the slots' int32 row ids, and
    per touched row the Q8_0 row read + write (2 x 136 B), the fp32 moments read +
    write (4 x 512 B) and the fp32 master read + write (2 x 512 B)."""
    return positions * 2 * WIDTH + positions * SLOTS * 4 + n_unique * (2 * Q8_ROW_BYTES + 4 * 512 + 2 * 512)


def bench_backward(tab, tokens, steps: int, warmup: int, cpu_s: float = 0.0) -> dict:
    """d_residual [16384, 2048] bf16 ~ N(0, 1e-3); scatter of
    the per-slot row gradients into the fp32 overlay of the touched rows (slots
    grouped per row, CSR, then each row's slots summed in slot order), Adam (lr
    1e-3, betas 0.9/0.999, eps 1e-8) on the touched rows and requantisation to
    Q8_0 blocks.  One step = one eg_descent_step call (a handful of launches)."""
    import torch

    from engraft_ngram_amd import descent as D
    from engraft_ngram_amd import synthetic as S

    _, rows = tab.forward(tokens, None, seq_len=SEQ, return_rows=True)
    rows = rows[0].contiguous()
    # RES_SETS output gradients rotate (67 MB each: a repeat would sit in the Infinity Cache)
    d_res = [S.residual(rows.shape[0], WIDTH, seed=RES_SEED + 100 + i, device=tab.device, std=1e-3)
             for i in range(RES_SETS)]
    state = D.DescentState.from_rows(tab, rows)
    torch.cuda.synchronize()
    for i in range(warmup):
        state.step(d_res[i % RES_SETS], rows, lr=1e-3)
    rot = itertools.count()
    ramp(lambda: state.step(d_res[next(rot) % RES_SETS], rows, lr=1e-3), 0.3)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(steps):
        state.step(d_res[i % RES_SETS], rows, lr=1e-3)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / steps
    nb = backward_bytes(rows.shape[0], state.n)
    gbs = nb / (ms * 1e-3) / 1e9
    # the same step from the slots' variables, as the forward over the state's
    # overlay writes them (eg_forward_slots; OverlayEmb's idx_r): no row lookup
    from engraft_ngram_amd import table as T
    fwd = T.PreparedForward([tab], tokens, None, overlays=[state.overlay()], seq_len=SEQ, return_slot_vars=True)
    fwd()
    sv = fwd.slot_vars[0]
    del fwd
    rot = itertools.count()
    ramp(lambda: state.step(d_res[next(rot) % RES_SETS], slot_var=sv, lr=1e-3), 0.3)
    a.record()
    for i in range(steps):
        state.step(d_res[i % RES_SETS], slot_var=sv, lr=1e-3)
    b.record()
    torch.cuda.synchronize()
    ms_sv = a.elapsed_time(b) / steps
    s1 = D.DescentState(state.ids, state.master.clone(), base=state.base)
    s2 = D.DescentState(state.ids, state.master.clone(), base=state.base)
    for i in range(2):
        s1.step(d_res[i], slot_var=sv, lr=1e-3)
        s2.step(d_res[i], rows, lr=1e-3)
    torch.cuda.synchronize()
    sv_same = bool(torch.equal(s1.master, s2.master) and torch.equal(s1.m, s2.m) and torch.equal(s1.v, s2.v)
                   and torch.equal(s1.quant.payload, s2.quant.payload))
    del s1, s2
    out = {"us_per_step": ms * 1e3, "touched_rows": state.n, "slot_gradients": rows.numel(),
           "algorithmic_bytes_per_step": nb, "gb_per_s": gbs, "frac_of_hbm_peak": gbs / HBM_PEAK_GBS,
           "us_per_step_from_slot_vars": ms_sv * 1e3,
           "frac_of_hbm_peak_from_slot_vars": nb / (ms_sv * 1e-3) / 1e9 / HBM_PEAK_GBS,
           "slot_vars_step_matches_rows_step": sv_same,
           "from_slot_vars": "the same step with each slot's variable given (what the forward over the state's "
                             "overlay writes, eg_forward_slots; the reference's OverlayEmb backward scatters by "
                             "these idx_r): the grouping needs no row lookup (eg_descent_plan_slots)",
           "rows_per_s": rows.numel() / (ms * 1e-3),
           "workload": "BASELINE config 2: scatter (CSR grouping + slot-ordered segmented reduce) + sparse Adam + "
                       "Q8_0 requant, fp32 master/m/v kept"}
    if cpu_s > 0:
        out["cpu_baseline"] = cpu_descent(tab, rows, d_res[0], cpu_s)
        out["cpu_baseline"]["gpu_speedup"] = out["rows_per_s"] / out["cpu_baseline"]["value"]
    return out


def cpu_descent(tab, rows, d_res, budget_s: float) -> dict:
    """The descent step on the host as the reference's CPU torch path runs it,
    on the full config-2 inputs (all 16,384 positions): ``index_add_`` of the
    slot gradients into the touched rows, ``torch.optim.Adam``, Q8_0
    requantisation, on every thread torch uses; its first step is compared with
    the device's first step from the same rows (relative error per row)."""
    import numpy as np
    import torch

    from engraft_ngram_amd import descent as D
    from oracle import cpu_baseline as CB

    rows_c = rows.cpu()
    d_c = d_res.cpu()
    ids = torch.unique(rows_c.reshape(-1).to(torch.int64))
    param0 = tab.gather(ids.to(torch.int32).to(tab.device).reshape(-1, 1)).float().cpu().reshape(ids.numel(), -1)
    td = CB.TorchDescent(rows_c, param0, lr=1e-3)
    td.step(d_c)
    fresh = D.DescentState.from_rows(tab, rows)
    fresh.step(d_res, rows, lr=1e-3)
    dev_p = fresh.master.cpu().numpy()
    cpu_p = td.param.detach().numpy()
    scale = np.maximum(np.abs(dev_p).max(axis=1, keepdims=True), 1e-30)
    rel = float((np.abs(cpu_p - dev_p) / scale).max())
    del fresh
    td = CB.TorchDescent(rows_c, param0, lr=1e-3)
    n, el = repeat_for(lambda: td.step(d_c), budget_s)
    threads = torch.get_num_threads()
    return {"value": n * rows_c.numel() / el, "unit": "slot gradients/s", "cores": threads, "kind": "port",
            "host": host_cpu(), "first_step_max_rel_err_vs_gpu": rel,
            "sample": f"full config-2 step ({rows_c.numel()} slots, {ids.numel()} rows) x {n} in {el:.1f} s: "
                      f"torch index_add_ + torch.optim.Adam + Q8_0 requant on {threads} threads"}


def bench_decode(tab, steps: int) -> dict:
    """the config-1 table plus a 500,000-row Q8_0 overlay
    (sorted ids, seeded rows), 256 sequences x (2 context tokens + 1 new); one
    eg_forward_decode per step, latency per call from HIP events around it."""
    import numpy as np
    import torch

    from engraft_ngram_amd import synthetic as S
    from engraft_ngram_amd import table as T
    from engraft_ngram_amd.overlay import DeviceOverlay

    dev = tab.device
    time.sleep(0.5)  # per-call latency: after the host threads of the CPU leg before it are idle
    n_seq, ctx, n_ov = 256, 3, 500_000
    ids = np.unique(np.random.default_rng(DECODE_SEED).integers(0, N_ROWS, size=n_ov + 4096))[:n_ov]
    store = T.RowStore.empty("q8_0", ids.size, DIM, dev)
    T.fill_synthetic(store, seed=DECODE_SEED + 1, sigma=0.02)
    ov = DeviceOverlay(torch.from_numpy(ids.astype(np.int32)).to(dev), store)
    # a new token per sequence at every step: 64 token sets rotate
    toks = [torch.from_numpy(S.zipf_tokens(DECODE_SEED + 2 + 7919 * j, n_seq * ctx, VOCAB).reshape(n_seq, ctx)).to(dev)
            for j in range(64)]
    res = S.residual(n_seq, WIDTH, seed=DECODE_SEED + 3, device=dev)
    out = torch.empty_like(res)
    ov_bm = DeviceOverlay(ov.ids, store).with_bitmap(tab.n_rows)

    def latencies(overlay) -> list:
        calls = [T.PreparedForward([tab], tk, res, out=out, overlays=[overlay], decode_ctx=ctx) for tk in toks]
        run = [c for c in calls]
        for i in range(200):
            run[i % 64]()
        rot = itertools.count()
        ramp(lambda: run[next(rot) % 64](), 0.2)
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        for i, (a, b) in enumerate(evs):
            a.record()
            run[i % 64]()
            b.record()
        torch.cuda.synchronize()
        return sorted(a.elapsed_time(b) * 1e3 for a, b in evs)

    def per_step_in_graphs(overlay, k: int = 16) -> list:
        """A decode loop of k steps (k token sets in turn) captured as one HIP
        graph; per-step time of each replay (replay time / k)."""
        calls = [T.PreparedForward([tab], tk, res, out=out, overlays=[overlay], decode_ctx=ctx) for tk in toks]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for c in calls:
                c()
        torch.cuda.current_stream().wait_stream(side)
        gs = []
        for j in range(0, len(calls), k):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for c in calls[j:j + k]:
                    c()
            gs.append(g)
        for i in range(20):
            gs[i % len(gs)].replay()
        rot = itertools.count()
        ramp(lambda: gs[next(rot) % len(gs)].replay(), 0.2, 5)
        n_rep = max(20, steps // k)
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n_rep)]
        for i, (a, b) in enumerate(evs):
            a.record()
            gs[i % len(gs)].replay()
            b.record()
        torch.cuda.synchronize()
        return sorted(a.elapsed_time(b) * 1e3 / k for a, b in evs)

    lat_search = latencies(ov)
    lat = latencies(ov_bm)
    lat_graph16 = per_step_in_graphs(ov_bm)
    pct = lambda v, q: v[min(len(v) - 1, int(len(v) * q))]
    nbytes = n_seq * (SLOTS * Q8_ROW_BYTES + 2 * 2 * WIDTH + ctx * 8)
    return {"workload": "BASELINE config 3: 256 sequences x (2 context + 1 new token), config-1 table + "
                        "500,000-row Q8_0 overlay resolved per id through its rank bitmap (Bloom filter + "
                        "per-word bits and ranks)",
            "calls": steps, "us_p50": pct(lat, 0.5), "us_p99": pct(lat, 0.99), "us_min": lat[0],
            "us_p50_binary_search": pct(lat_search, 0.5), "us_p99_binary_search": pct(lat_search, 0.99),
            "us_per_step_p50_graph_of_16_steps": pct(lat_graph16, 0.5),
            "us_per_step_p99_graph_of_16_steps": pct(lat_graph16, 0.99),
            "lookups_per_call": n_seq * SLOTS, "algorithmic_bytes_per_call": nbytes}


def bench_config4(steps: int, warmup: int) -> dict:
    """2 table layers x 160,000,000 MXFP8 rows, 2-/3-/4-gram
    hashes (24 slots per layer), 32,768 Zipf tokens over 129,280, residual width
    3,072; one fused launch per step (both layers summed in fp32)."""
    import torch

    from engraft_ngram_amd import synthetic as S
    from engraft_ngram_amd import table as T

    dev = torch.device("cuda", 0)
    rows4, seq4, vocab4, width4, slots4 = 160_000_000, 32_768, 129_280, 3072, 24
    tabs = []
    for l in range(2):
        hp = S.hash_params(rows4, C4_SEED + l, ngram_size=4)
        tabs.append(T.DeviceTable.synthetic("mxfp8", rows4, DIM, seed=C4_SEED + 10 + l, sigma=0.02, device=dev,
                                            **hp))
    tok = torch.from_numpy(S.zipf_tokens(C4_SEED + 20, seq4, vocab4)).to(dev)
    res = [S.residual(seq4, width4, seed=C4_SEED + 30 + i, device=dev) for i in range(2)]
    outs = [torch.empty_like(r) for r in res]
    # 8 token batches rotate (each call a new batch), the two residual sets with them
    toks = [tok] + [torch.from_numpy(S.zipf_tokens(C4_SEED + 20 + 1000 * j, seq4, vocab4)).to(dev) for j in range(1, 8)]
    calls = [T.PreparedForward(tabs, toks[i], res[i % 2], out=outs[i % 2]) for i in range(8)]
    for i in range(warmup):
        calls[i % 8]()
    rot = itertools.count()
    ramp(lambda: calls[next(rot) % 8](), 0.3)
    ev = _Events(4)
    torch.cuda.synchronize()
    for i in range(steps):
        c = calls[i % 8]
        if i == 0:
            c.timed(ev[0], ev[1] if steps > 1 else ev[3])
        elif i == steps - 1:
            c.timed(ev[2], ev[3])
        else:
            c()
    torch.cuda.synchronize()
    us = ev.elapsed_ms(0, 3) / steps * 1e3
    ev.destroy()
    row_bytes = DIM + DIM // 32  # e4m3 values + e8m0 scales
    nbytes = seq4 * (2 * slots4 * row_bytes + 2 * 2 * width4 + 8)
    gbs = nbytes / (us * 1e-6) / 1e9
    del tabs
    torch.cuda.empty_cache()
    return {"workload": "BASELINE config 4: 2 layers x 160M MXFP8 rows, 24 slots/layer, seq 32768, width 3072",
            "us_per_launch": us, "rows_per_s": seq4 * 2 * slots4 / (us * 1e-6), "gb_per_s": gbs,
            "frac_of_hbm_peak": gbs / HBM_PEAK_GBS, "algorithmic_bytes_per_launch": nbytes}


def bench_real_format(steps: int, warmup: int) -> dict:
    """The reference's own table format (the f4 path, engraft/table.py:40-169):
    16 heads x 20,000,096 rows of 160 values in IQ4_NL blocks (90 B per row,
    28.8 GB as the file holds them), the reference's hash mode (three multipliers shared by every head),
    16,384 Zipf tokens per step into a bf16 residual [16384, 2560]; 16 token
    batches and 4 residual sets rotate.  Rows: random nibbles, block scale
    fp16(0.002).  The rows sit in 128-byte lines of their own (PleTable's
    default layout): one line per random row read.  Algorithmic bytes count
    the 90 bytes of a row."""
    import numpy as np
    import torch

    from engraft_ngram_amd import synthetic as S
    from engraft_ngram_amd import table as T

    dev = torch.device("cuda", 0)
    per, heads, dim = 20_000_096, 16, 160
    n_rows, width = per * heads, heads * dim
    store = T.RowStore.empty("iq4_nl", n_rows, dim, dev, row_stride=T.RowStore.padded_stride("iq4_nl", dim))
    g = torch.Generator(device=dev).manual_seed(REAL_SEED)
    chunk = 1 << 26
    scale = np.array([0.002], dtype=np.float16).view(np.uint8)
    for r0 in range(0, n_rows, chunk):
        blk = store.payload[r0:r0 + chunk]
        blk.random_(0, 256, generator=g)
        v = blk[:, :store.row_bytes].unflatten(1, (dim // 32, 18))
        v[:, :, 0] = int(scale[0])
        v[:, :, 1] = int(scale[1])
    mults = [int(m) for m in S.odd_multipliers(REAL_SEED, 3)]
    tab = T.DeviceTable(store, eos_token_id=S.QWEN_EOS, ngram_size=3, heads_per_ngram=8, layer_multipliers=mults,
                        head_vocab_sizes=[per] * heads, head_offsets=[h * per for h in range(heads)])
    n_pos = BATCH * SEQ
    toks = [torch.from_numpy(S.zipf_tokens(REAL_SEED + 1 + 1000 * j, n_pos, VOCAB)).to(dev) for j in range(TOKEN_SETS)]
    res = [S.residual(n_pos, width, seed=REAL_SEED + 50 + i, device=dev) for i in range(RES_SETS)]
    outs = [torch.empty_like(r) for r in res]
    n_sets = max(TOKEN_SETS, RES_SETS)
    calls = [T.PreparedForward([tab], toks[i % TOKEN_SETS], res[i % RES_SETS], out=outs[i % RES_SETS], seq_len=SEQ)
             for i in range(n_sets)]
    for i in range(warmup):
        calls[i % n_sets]()
    rot = itertools.count()
    ramp(lambda: calls[next(rot) % n_sets](), 0.3)
    ev = _Events(4)
    torch.cuda.synchronize()
    for i in range(steps):
        c = calls[i % n_sets]
        if i == 0:
            c.timed(ev[0], ev[1] if steps > 1 else ev[3])
        elif i == steps - 1:
            c.timed(ev[2], ev[3])
        else:
            c()
    torch.cuda.synchronize()
    us = ev.elapsed_ms(0, 3) / steps * 1e3
    ev.destroy()
    nbytes = n_pos * (heads * 90 + 2 * 2 * width + 8)
    gbs = nbytes / (us * 1e-6) / 1e9
    del tab, store
    torch.cuda.empty_cache()
    return {"workload": "the reference's real table format: 16 heads x 20,000,096 IQ4_NL rows of 160 (90 B, each in "
                        "a 128-byte line of its own), "
                        "shared multipliers, 16,384 Zipf tokens, residual width 2560",
            "us_per_launch": us, "rows_per_s": n_pos * heads / (us * 1e-6), "gb_per_s": gbs,
            "frac_of_hbm_peak": gbs / HBM_PEAK_GBS, "algorithmic_bytes_per_launch": nbytes}


def bench_damage_scan(tab, steps: int, hp: dict | None = None, cpu_s: float = 0.0) -> dict:
    """The damage scan (the f3 path, engraft/damage.py:159-224): one corpus block
    of 8,000,000 Zipf tokens (the reference's block size, damage.py:60) against
    500,000 sorted overlay rows with their dnorm, on the config-1 table's hash:
    the fused eg_scan_overlay launch on device-resident tokens (HIP events),
    and damage.scan_hits end to end per block over a 32M-token corpus (tokens
    from the host, hit lists back)."""
    import ctypes

    import numpy as np
    import torch

    from engraft_ngram_amd import _lib, damage
    from engraft_ngram_amd import synthetic as S

    dev = tab.device
    n = 8_000_000
    tokens = S.zipf_tokens(SCAN_SEED, n, VOCAB)
    rng = np.random.default_rng(SCAN_SEED + 1)
    ids = np.unique(rng.integers(0, N_ROWS, size=520_000))[:500_000].astype(np.int32)
    dnorm = rng.random(ids.size).astype(np.float32)
    tok = torch.from_numpy(tokens).to(dev)
    ids_d, dn_d = torch.from_numpy(ids).to(dev), torch.from_numpy(dnorm).to(dev)
    n_hit = torch.empty(n, dtype=torch.int32, device=dev)
    dmax, dsum = torch.empty(n, device=dev), torch.empty(n, device=dev)
    counts = torch.zeros(ids.size, dtype=torch.int64, device=dev)
    spec = tab.c_spec
    n_bits = tab.n_rows
    bitmap = torch.empty(int(_lib.load().eg_id_bitmap_words(n_bits)), dtype=torch.int32, device=dev)
    _lib.call("eg_build_id_bitmap", _lib.ptr(ids_d), ids.size, _lib.ptr(bitmap), n_bits, _lib.stream_ptr(dev))

    def timed(bm) -> float:
        args = (ctypes.byref(spec), _lib.ptr(tok), 8, n, 0, _lib.ptr(ids_d), ids.size, bm, n_bits, _lib.ptr(dn_d),
                _lib.ptr(n_hit), _lib.ptr(dmax), _lib.ptr(dsum), _lib.ptr(counts), _lib.stream_ptr(dev))
        for _ in range(3):
            _lib.call("eg_scan_overlay", *args)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            _lib.call("eg_scan_overlay", *args)
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / steps * 1e3

    us_search = timed(None)
    us = timed(_lib.ptr(bitmap))
    counts.zero_()
    _lib.call("eg_scan_overlay", ctypes.byref(spec), _lib.ptr(tok), 8, n, 0, _lib.ptr(ids_d), ids.size,
              _lib.ptr(bitmap), n_bits, _lib.ptr(dn_d), _lib.ptr(n_hit), _lib.ptr(dmax), _lib.ptr(dsum),
              _lib.ptr(counts), _lib.stream_ptr(dev))
    counts_ref = counts.cpu().numpy()
    # end to end over a four-block corpus (32M tokens): block i+1 uploads while block i is scanned.
    # The first full call pins the host staging buffers (kept by torch's host allocator); the
    # median of three calls after it is the steady state of a long corpus.
    corpus = np.concatenate([tokens] + [S.zipf_tokens(SCAN_SEED + 10 + i, n, VOCAB) for i in range(3)])
    corpus32 = corpus.astype(np.int32)  # a tokenized corpus file's int32 ids

    def end_to_end(toks):
        damage.scan_hits(toks, tab, ids, dnorm)
        walls = []
        for _ in range(3):
            t0 = time.perf_counter()
            r = damage.scan_hits(toks, tab, ids, dnorm)
            walls.append((time.perf_counter() - t0) / 4)
        return r, float(np.median(walls))

    res, wall = end_to_end(corpus)
    res32, wall32 = end_to_end(corpus32)
    assert np.array_equal(res32["pos"], res["pos"]) and np.array_equal(res32["read_count"], res["read_count"])
    lookups = n * tab.n_heads
    # algorithmic bytes of one block: each token read once (8 B), the three
    # per-position outputs written (4 B each), every overlay row's read count
    # read and written (8 + 8 B) and its dnorm read (4 B); the filter, pairs
    # and hash parameters are the lookup structure's own traffic
    algo = n * (8 + 12) + ids.size * (8 + 8 + 4)
    out = {"workload": "damage scan: 8,000,000 Zipf tokens x 16 rows against 500,000 sorted overlay rows",
           "us_per_block_kernel": us, "us_per_block_kernel_search_only": us_search,
           "algorithmic_bytes_per_block": algo, "gb_per_s": algo / (us * 1e-6) / 1e9,
           "frac_of_hbm_peak": algo / (us * 1e-6) / (HBM_PEAK_GBS * 1e9),
           "traffic_bytes_per_block": traffic_from_profile("damage_scan_bitmap"),
           "tokens_per_s_kernel": n / (us * 1e-6), "lookups_per_s_kernel": lookups / (us * 1e-6),
           "s_per_block_end_to_end": wall, "s_per_block_end_to_end_int32_tokens": wall32,
           "hit_positions": int(res["pos"].size)}
    if cpu_s > 0 and hp is not None:
        from concurrent.futures import ThreadPoolExecutor

        from oracle import cpu_baseline as CB
        spec = oracle_spec(hp)
        threads = torch.get_num_threads()
        with ThreadPoolExecutor(threads) as pool:
            k, el = repeat_for(lambda: CB.scan_block_threads(spec, tokens, ids, dnorm, threads, pool), cpu_s)
            r = CB.scan_block_threads(spec, tokens, ids, dnorm, threads, pool)
        same = bool(np.array_equal(r["read_count"], counts_ref)) if counts_ref is not None else None
        out["cpu_baseline"] = {"value": k * n / el, "unit": "tokens/s", "cores": threads, "kind": "port",
                               "host": host_cpu(), "read_counts_match_gpu": same,
                               "sample": f"the full 8,000,000-token block x {k} in {el:.1f} s: vectorized numpy "
                                         f"hash + searchsorted + bincount, split over {threads} threads"}
        out["cpu_baseline"]["gpu_speedup"] = out["tokens_per_s_kernel"] / out["cpu_baseline"]["value"]
    return out


def bench_overlay_emb(tab, steps: int, hp: dict | None = None, cpu_s: float = 0.0) -> dict:
    """The differentiable overlay of the descent loop (a8, OverlayEmb,
    engraft/replica/seq.py:237-444): one 2,048-token Zipf sequence on the
    config-1 table, 14,032 of its rows as fp32 variables (the size of the
    reference's Quail s0b overlay, docs/formats.md:120-124); a step is build()
    (the cached plan's gather with the variables substituted) plus the backward
    of a given upstream gradient into the variables (what the model's backward
    hands the embedding).  CPU: the reference's step with the plan cached
    (torch index_put into the base rows + autograd backward of the same
    gradient) on every host thread."""

    import ctypes

    import numpy as np
    import torch

    from engraft_ngram_amd import synthetic as S
    from engraft_ngram_amd.seq import OverlayEmb

    dev = tab.device
    # a host-bound step: time it after the host threads of earlier CPU legs
    # (thread pools, BLAS and OpenMP workers that spin after their work) are idle
    time.sleep(0.5)
    t_len, n_var = 2048, 14_032
    tokens = S.zipf_tokens(SCAN_SEED + 2, t_len, VOCAB)
    rows = tab.rows(torch.from_numpy(tokens).to(dev), seq_len=t_len).cpu().numpy()
    uniq = np.unique(rows.reshape(-1))
    pick = np.sort(np.random.default_rng(SCAN_SEED + 3).choice(uniq, size=min(n_var, uniq.size), replace=False))
    row_map = {int(g): i for i, g in enumerate(pick)}
    rv = tab.gather(torch.from_numpy(pick.astype(np.int32)).to(dev).reshape(-1, 1)).float()
    rv = rv.reshape(pick.size, -1).contiguous().requires_grad_(True)
    oe = OverlayEmb(tab, tokens.tolist(), rv, row_map)
    g = torch.randn((t_len, tab.n_heads * DIM), generator=torch.Generator(device=dev).manual_seed(5), device=dev)

    def step():
        rv.grad = None
        oe.build(t_len).backward(g)

    step()  # plans the sequence once, as the reference's overlay_cache does
    # a host-bound step: timed in steady state, after a fifth of a second of
    # steps (the host cores at speed) and over at least 1,000 steps
    steps = max(steps, 1000)
    repeat_for(step, 0.2)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        step()
    b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) / steps * 1e3
    # The same steps with autograd's backward run on the calling thread (torch's
    # thread-local switch; by default the engine hands a CUDA backward to its
    # device thread and waits for it).
    with torch.autograd.set_multithreading_enabled(False):
        repeat_for(step, 0.2)
        torch.cuda.synchronize()
        a.record()
        for _ in range(steps):
            step()
        b.record()
        torch.cuda.synchronize()
    us_calling_thread = a.elapsed_time(b) / steps * 1e3
    hits = int(oe.n_id_hits)
    # The device's share of the step: the same two launches (eg_gather_slots over
    # the cached plan, eg_scatter_grad_apply from its cached grouping) issued back
    # to back without torch autograd around them.  The wall figure above also
    # holds autograd's own host work (its device thread hand-offs), which varies
    # from box to box several-fold for the same kernels.
    from engraft_ngram_amd import _lib
    from engraft_ngram_amd.seq import _slot_grouping

    plan = oe._plans[(0, t_len)]
    ws = _slot_grouping(plan, pick.size, dev)
    emb = torch.empty((t_len, tab.n_heads * DIM), dtype=torch.float32, device=dev)
    grad = torch.empty((pick.size, DIM), dtype=torch.float32, device=dev)
    lib = _lib.load()
    st = torch.cuda.current_stream(dev).cuda_stream
    ct = tab.c_table
    rvd = rv.detach()

    def device_step():
        lib.eg_gather_slots(ctypes.byref(ct), plan["rows"].data_ptr(), plan["slot_var"].data_ptr(), t_len,
                            tab.n_heads, rvd.data_ptr(), pick.size, emb.data_ptr(), st)
        lib.eg_scatter_grad_apply(g.data_ptr(), 1, t_len, tab.n_heads, DIM, pick.size, grad.data_ptr(), 1,
                                  ws.data_ptr(), ws.numel(), st)

    device_step()
    torch.cuda.synchronize()
    assert torch.equal(emb, oe.build(t_len).detach()) and torch.equal(grad, rv.grad)
    for _ in range(50):
        device_step()
    a.record()
    for _ in range(steps):
        device_step()
    b.record()
    torch.cuda.synchronize()
    dev_us = a.elapsed_time(b) / steps * 1e3
    out = {"workload": "OverlayEmb: 2,048-token sequence, config-1 table, 14,032 fp32 variable rows; build + backward",
           "us_per_step": us, "positions_per_s": t_len / (us * 1e-6), "slots_replaced": hits,
           "us_per_step_backward_on_calling_thread": us_calling_thread,
           "device_us_per_step": dev_us,
           "device_us_per_step_note": "eg_gather_slots + eg_scatter_grad_apply back to back (the step's kernels, "
                                      "outputs checked equal to the autograd step's); us_per_step adds torch "
                                      "autograd's host work around them (build() and the backward are C++ autograd "
                                      "code; torch's engine runs a CUDA backward on its device thread, and "
                                      "us_per_step_backward_on_calling_thread is the same step under "
                                      "torch.autograd.set_multithreading_enabled(False))"}
    if cpu_s > 0 and hp is not None:
        # The reference's step on the CPU with the plan cached (seq.py:428-444):
        # base.index_put((idx_t, idx_h), rows_var[idx_r]) and the autograd
        # backward into rows_var, torch on every host thread, the whole
        # sequence.  The cached plan (row ids, base rows, substitution indices)
        # is built once from the device's row ids and base gather.
        base = tab.gather(torch.as_tensor(rows.reshape(-1, 1).astype(np.int32), device=dev)).float().cpu()
        base = base.reshape(t_len, tab.n_heads, -1)
        hit = np.isin(rows, pick)
        it_np, ih_np = np.nonzero(hit)
        ir_np = np.searchsorted(pick, rows[it_np, ih_np])
        it_t, ih_t, ir_t = (torch.from_numpy(x.astype(np.int64)) for x in (it_np, ih_np, ir_np))
        rv_c = rv.detach().cpu().clone().requires_grad_(True)
        g_c = g.cpu().reshape(t_len, tab.n_heads, -1)

        def cpu_step():
            rv_c.grad = None
            base.index_put((it_t, ih_t), rv_c[ir_t]).backward(g_c)

        cpu_step()
        step()
        torch.cuda.synchronize()
        ref = rv.grad.detach().cpu()
        err = float((rv_c.grad - ref).abs().max() / ref.abs().max().clamp_min(1e-30))
        k, el = repeat_for(cpu_step, cpu_s)
        out["cpu_baseline"] = {"value": k * t_len / el, "unit": "positions/s", "cores": torch.get_num_threads(),
                               "kind": "port", "host": host_cpu(),
                               "grad_max_rel_err_vs_gpu": err,
                               "sample": f"the whole {t_len}-token sequence x {k} in {el:.1f} s, plan cached as the "
                                         "reference caches it: torch index_put of the variables into the cached base "
                                         "rows + autograd backward into them (seq.py:428-444), "
                                         f"{torch.get_num_threads()} threads",
                               "gpu_speedup": out["positions_per_s"] / (k * t_len / el)}
    return out


def bench_ple(steps: int, warmup: int, cpu_s: float = 0.0) -> dict:
    """The PLE block consuming the rows (engraft/replica/layers.py:565-626) at
    the real model's dimensions: 2048 positions, 4 hyper-connection streams,
    n_embd 2560, 4 conv taps with dilation 3; seeded random weights; fp32."""
    import torch

    from engraft_ngram_amd import ple

    class HP:
        hc_mult, n_embd, f_norm_rms_eps, ple_ngram_size = 4, 2560, 1e-6, 3

    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(PLE_SEED)
    hc, n, t_len = 4, 2560, 2048
    rnd = lambda *shape, sc=1.0: torch.randn(shape, generator=g, device=dev) * sc
    w = ple.PleWeights(w_key=rnd(hc * n, n, sc=n ** -0.5), w_value=rnd(n, n, sc=n ** -0.5),
                       norm_key=1 + rnd(hc * n, sc=0.1), norm_query=1 + rnd(hc * n, sc=0.1),
                       norm_conv=1 + rnd(hc * n, sc=0.1), conv1d=rnd(hc * n, 4, sc=0.5))
    emb, hidden = rnd(t_len, n, sc=0.1), rnd(t_len, hc, n, sc=0.1)
    hist = torch.zeros(0, hc, n, device=dev)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn, k: int) -> float:
        torch.cuda.synchronize()
        a.record()
        for _ in range(k):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / k

    flops = 2.0 * t_len * n * (hc * n + n)
    d_out = rnd(t_len, hc, n, sc=1e-3)
    emb_v = emb.clone().requires_grad_(True)
    res = {}
    for mode in ("fp32", "bf16x3", "bf16x6"):
        with torch.no_grad():
            for _ in range(warmup):
                ple.ple_forward(emb, hidden, w, hist, HP, gemm=mode)
            ramp(lambda: ple.ple_forward(emb, hidden, w, hist, HP, gemm=mode), 0.3)
            ms = timed(lambda: ple.ple_forward(emb, hidden, w, hist, HP, gemm=mode), steps)
            # the two projections alone (one launch, as ple_forward runs them), for the GEMMs' own rate
            if mode == "fp32":
                gemm_ms = timed(lambda: ple.gemm_f32(emb, w.w_key, b_n2=w.w_value), steps)
                # the same products through hipBLASLt (torch.matmul, no TF32), for reference
                allow = torch.backends.cuda.matmul.allow_tf32
                torch.backends.cuda.matmul.allow_tf32 = False
                lib = lambda: (emb @ w.w_key.T, emb @ w.w_value.T)
                ramp(lib, 0.3)  # its first calls under a new setting pick and load kernels
                lib_ms = timed(lib, steps)
                torch.backends.cuda.matmul.allow_tf32 = allow
            elif mode == "bf16x3":
                pk, pv = ple.SplitPlanes(w.w_key), ple.SplitPlanes(w.w_value)
                gemm_ms = timed(lambda: ple.gemm_x3(emb, pk, b_n2=pv), steps)
            else:
                pk, pv = ple.SplitPlanes(w.w_key, three=True), ple.SplitPlanes(w.w_value, three=True)
                gemm_ms = timed(lambda: ple.gemm_x6(emb, pk, b_n2=pv), steps)
        # forward + backward to emb (the descent's use: the weights stay fixed)
        fb = lambda: torch.autograd.grad(ple.ple_forward(emb_v, hidden, w, hist, HP, gemm=mode)[0], emb_v, d_out)
        fb()
        ramp(fb, 0.2, 3)
        fb_ms = timed(fb, max(10, steps // 2))
        res[mode] = {"us_per_step": ms * 1e3, "positions_per_s": t_len / (ms * 1e-3), "gemm_us": gemm_ms * 1e3,
                     "gemm_tflops": flops / (gemm_ms * 1e-3) / 1e12, "non_gemm_us": (ms - gemm_ms) * 1e3,
                     "us_forward_backward_to_emb": fb_ms * 1e3}
        if mode == "fp32":
            res[mode]["hipblaslt_gemm_us"] = lib_ms * 1e3
            res[mode]["hipblaslt_gemm_tflops"] = flops / (lib_ms * 1e-3) / 1e12
    # each GEMM's largest error against the float64 products, relative to
    # |emb| |W|^T (the scale of an fp32 sum's rounding), key and value together
    with torch.no_grad():
        e64 = emb.double()
        refs = [(e64 @ x.double().T, e64.abs() @ x.double().abs().T) for x in (w.w_key, w.w_value)]

        def err(outs) -> float:
            return max(float(((o.double() - r).abs() / (bd + 1e-30)).max()) for o, (r, bd) in zip(outs, refs))

        allow = torch.backends.cuda.matmul.allow_tf32
        torch.backends.cuda.matmul.allow_tf32 = False
        errs = {"fp32": err(ple.gemm_f32(emb, w.w_key, b_n2=w.w_value)),
                "hipblaslt": err((emb @ w.w_key.T, emb @ w.w_value.T)),
                "bf16x3": err(ple.gemm_x3(emb, w.w_key, b_n2=w.w_value)),
                "bf16x6": err(ple.gemm_x6(emb, w.w_key, b_n2=w.w_value))}
        torch.backends.cuda.matmul.allow_tf32 = allow
        del refs, e64
    res["fp32"]["gemm_err_vs_fp64"] = errs["fp32"]
    res["fp32"]["hipblaslt_gemm_err_vs_fp64"] = errs["hipblaslt"]
    res["bf16x3"]["gemm_err_vs_fp64"] = errs["bf16x3"]
    res["bf16x6"]["gemm_err_vs_fp64"] = errs["bf16x6"]
    out = {"workload": "ple_forward: T 2048, hc 4, n_embd 2560, 4 taps, dilation 3, fp32 activations; key/value "
                       "GEMMs (one launch) either fp32 (eg_gemm_f32 on the fp32 matrix cores; the reference's "
                       "arithmetic; hipBLASLt's time for the same products beside it), bf16x3 (eg_gemm_bf16x3 "
                       "on the bf16 matrix cores, 16 mantissa bits per operand) or bf16x6 (eg_gemm_bf16x6: three "
                       "bf16 planes an operand, six products, fp32 accuracy; ple_forward's default); gate/norm "
                       "and conv in HIP; gemm_err_vs_fp64: the largest |C - C64| / (|emb| |W|^T); the top-level "
                       "figures are the fp32 mode's",
           **res["fp32"], "default_gemm": "bf16x6", "bf16x3": res["bf16x3"], "bf16x6": res["bf16x6"],
           "fp32_mfma_peak_tflops": 157.3,
           "bf16_mfma_peak_tflops": 2500.0}
    if cpu_s > 0:
        from oracle import ple as OP
        tc = 256
        wc = {k: getattr(w, k).cpu() for k in ("w_key", "w_value", "norm_key", "norm_query", "norm_conv", "conv1d")}
        ec, hcpu = emb[:tc].cpu(), hidden[:tc].cpu()
        with torch.no_grad():
            k, el = repeat_for(lambda: OP.ple_forward(ec, hcpu, wc, hist.cpu(), hc, n, 1e-6, 3), cpu_s)
        out["cpu_baseline"] = {"value": k * tc / el, "unit": "positions/s", "cores": torch.get_num_threads(),
                               "kind": "port",
                               "sample": f"first {tc} positions x {k} in {el:.1f} s: oracle ple_forward (torch "
                                         f"fp32 on the CPU, {torch.get_num_threads()} threads)"}
        out["cpu_baseline"]["gpu_speedup"] = out["positions_per_s"] / out["cpu_baseline"]["value"]
    return out


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=2000)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="CPU baseline time budget")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-backward", action="store_true", help="skip the config-2 descent step leg")
    ap.add_argument("--no-extra", action="store_true", help="skip the config-3 decode and config-4 legs")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 1 GiB device copy (torch copy_) 10 times: the known-size kernel the "
                         "FETCH_SIZE / WRITE_SIZE counters are scaled by")
    ap.add_argument("--forward-table-rows", type=int, default=0,
                    help="only run the config-1 forward (same tokens, residual and hash seeds) over a table of "
                         "this many rows, 400 launches, and print its time: the table-size sweep behind the "
                         "forward's translation-reach measurements")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build measures the table path on one "
              "GPU (every box here has one MI355X). The path shards by positions (forward, table replicated) "
              "and by variable owner (backward); that layout is not built here.", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_calibration:
        src = torch.ones(1 << 28, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(10):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration": {"bytes_read": src.numel() * 4, "bytes_written": dst.numel() * 4,
                                               "launches": 10}}), flush=True)
        return

    pkg = __graft_entry__.load_package()
    from engraft_ngram_amd import synthetic as S
    from engraft_ngram_amd import table as T

    pkg._lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    n_pos = BATCH * SEQ

    if args.forward_table_rows:
        print(json.dumps({"forward_table_rows": forward_table_rows(args.forward_table_rows, dev)}), flush=True)
        return

    t0 = time.perf_counter()
    hp = S.hash_params(N_ROWS, HASH_SEED)
    tab = T.DeviceTable.synthetic("q8_0", N_ROWS, DIM, seed=TABLE_SEED, sigma=0.02, device=dev, **hp)
    torch.cuda.synchronize()
    log(f"table: {N_ROWS} rows q8_0 ({N_ROWS * Q8_ROW_BYTES / 1e9:.2f} GB) generated in "
        f"{time.perf_counter() - t0:.2f} s")
    # Every step is a new batch: TOKEN_SETS Zipf token batches and RES_SETS
    # residual/output sets rotate, so that neither the touched table rows
    # (≈ 62 MB of lines per batch) nor the residual (134 MB per step) is served
    # from the 256 MB Infinity Cache by a repeat of the previous steps.
    tokens_np = S.zipf_tokens(TOKEN_SEED, n_pos, VOCAB)
    tok_sets = [torch.from_numpy(tokens_np).to(dev)] + [
        torch.from_numpy(S.zipf_tokens(TOKEN_SEED + 1000 * j, n_pos, VOCAB)).to(dev) for j in range(1, TOKEN_SETS)]
    tokens = tok_sets[0]
    res = [S.residual(n_pos, WIDTH, seed=RES_SEED + i, device=dev) for i in range(RES_SETS)]
    outs = [torch.empty_like(r) for r in res]
    n_sets = max(TOKEN_SETS, RES_SETS)
    calls = [T.PreparedForward([tab], tok_sets[i % TOKEN_SETS], res[i % RES_SETS], out=outs[i % RES_SETS],
                               seq_len=SEQ) for i in range(n_sets)]
    torch.cuda.synchronize()

    # clock ramp (time-based, whatever --warmup is), then the W warm-up steps
    rot = itertools.count()
    ramp_calls = ramp(lambda: calls[next(rot) % n_sets](), 0.5)
    for i in range(args.warmup):
        calls[i % n_sets]()
    torch.cuda.synchronize()

    # ---- the timed region: exactly K steps, synchronised on both sides.  The
    # first and last launch go through eg_forward_timed, whose hipEvent_t pairs
    # take the dispatches' own timestamps on the launch stream: start of the
    # first kernel -> end of the last = K back-to-back launches. ----
    ev = _Events(4)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for i in range(args.steps):
        c = calls[i % n_sets]
        if i == 0:
            c.timed(ev[0], ev[1] if args.steps > 1 else ev[3])
        elif i == args.steps - 1:
            c.timed(ev[2], ev[3])
        else:
            c()
    end.record()
    torch.cuda.synchronize()
    ms_per_step = start.elapsed_time(end) / args.steps
    kernel_ms = ev.elapsed_ms(0, 3) / args.steps
    first_ms = ev.elapsed_ms(0, 1)
    ev.destroy()

    rows_per_step = n_pos * SLOTS
    fbytes = forward_bytes(n_pos)
    # the library's streaming copy moving the kernel's measured HBM traffic (profiles/), for scale
    traffic = traffic_from_profile("forward_q8_cfg1")
    copy_us = copy_ceiling_us(traffic, dev) if traffic else None
    if copy_us:
        log(f"forward: the streaming copy moving the same {traffic / 1e6:.1f} MB takes {copy_us:.1f} us")
    ceilings = stream_ceilings(dev)
    # the same step with the row ids given (eg_forward_rows): the forward without its hash
    rows_sets = [T.forward([tab], tok_sets[j], res[0], out=outs[0], seq_len=SEQ, return_rows=True)[1]
                 for j in range(TOKEN_SETS)]
    rcalls = [T.PreparedForwardRows([tab], rows_sets[i % TOKEN_SETS], res[i % RES_SETS], out=outs[i % RES_SETS])
              for i in range(n_sets)]
    rot = itertools.count()
    ramp(lambda: rcalls[next(rot) % n_sets](), 0.2)
    start.record()
    for i in range(args.steps):
        rcalls[i % n_sets]()
    end.record()
    torch.cuda.synchronize()
    hash_free_us = start.elapsed_time(end) / args.steps * 1e3
    del rcalls, rows_sets
    log(f"forward with the row ids given (no hash): {hash_free_us:.1f} us/launch")
    achieved = fbytes / (kernel_ms * 1e-3) / 1e9
    log(f"forward: {ms_per_step * 1e3:.1f} us/step wall, {kernel_ms * 1e3:.1f} us/launch back to back "
        f"(first launch alone {first_ms * 1e3:.1f}), {achieved:.0f} GB/s algorithmic")

    result = {
        "metric": METRIC,
        "value": rows_per_step / (ms_per_step * 1e-3),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded on the device: 320M-row Q8_0 table ~N(0,0.02), Zipf(1.1) tokens, bf16 "
                "residual ~N(0,1))",
        "config": {
            "workload": "BASELINE config 1 forward: hash (2- and 3-gram, 16 slots) + gather + Q8_0 dequant "
                        "+ bf16 residual add, one fused launch per step",
            "table_rows": N_ROWS, "dim": DIM, "row_format": "q8_0 split: 128 B int8 + 4 fp16 scales",
            "batch": BATCH, "seq_len": SEQ, "slots_per_position": SLOTS, "residual_width": WIDTH,
            "vocab": VOCAB, "zipf_s": 1.1, "token_batches_rotated": TOKEN_SETS, "residual_sets_rotated": RES_SETS,
        },
        "roofline": {
            "bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
            "kernel": "eg::forward_kernel<2, 128, 2, 1, false, false, 2, false> (Q8_0, dim 128, 2 x 1024-column parts per position, bf16 out, no overlay, hashing)",
            "algorithmic_bytes_per_launch": fbytes, "avg_launch_us": kernel_ms * 1e3,
            "copy_of_same_traffic_us": copy_us,
            "launch_vs_copy_of_same_traffic": (kernel_ms * 1e3 / copy_us) if copy_us else None,
            "hash_free_us": hash_free_us,
            "hash_free_frac": fbytes / (hash_free_us * 1e-6) / 1e9 / HBM_PEAK_GBS,
            "stream_ceilings": ceilings,
            "clock_ramp_calls": ramp_calls,
        },
        "forward": {
            "rows_per_s": rows_per_step / (kernel_ms * 1e-3),
            "gb_per_s": achieved,
            "table_gb_per_s": n_pos * SLOTS * Q8_ROW_BYTES / (kernel_ms * 1e-3) / 1e9,
            "us_per_launch": kernel_ms * 1e3, "us_first_launch": first_ms * 1e3,
            "us_per_step_wall": ms_per_step * 1e3,
        },
    }

    # the other legs' CPU baselines (the oracle on a bounded sample, a few seconds each)
    cpu_leg_s = 0.0 if args.no_cpu else min(4.0, args.cpu_seconds)
    if not args.no_backward:
        bw = bench_backward(tab, tokens, max(50, args.steps // 4), max(20, args.warmup // 4), cpu_leg_s)
        result["backward"] = bw
        log_cpu_leg("backward", bw)
        log(f"backward: {bw['us_per_step']:.1f} us/step, {bw['touched_rows']} touched rows, "
            f"{bw['gb_per_s']:.0f} GB/s algorithmic ({100 * bw['frac_of_hbm_peak']:.1f}% of peak); from the "
            f"forward's slot variables {bw['us_per_step_from_slot_vars']:.1f} us/step "
            f"({100 * bw['frac_of_hbm_peak_from_slot_vars']:.1f}% of peak, same bits: "
            f"{bw['slot_vars_step_matches_rows_step']})")

    if not args.no_extra:
        dc = bench_decode(tab, 200)
        result["decode_config3"] = dc
        log(f"decode (config 3): p50 {dc['us_p50']:.1f} us, p99 {dc['us_p99']:.1f} us per call (binary search in "
            f"place of the bitmap: p50 {dc['us_p50_binary_search']:.1f} us); 16 steps captured as one "
            f"graph: p50 {dc['us_per_step_p50_graph_of_16_steps']:.1f} us per step")
        c4 = bench_config4(max(50, args.steps // 4), max(20, args.warmup // 4))
        result["forward_config4"] = c4
        log(f"forward (config 4): {c4['us_per_launch']:.1f} us/launch, {c4['gb_per_s']:.0f} GB/s algorithmic "
            f"({100 * c4['frac_of_hbm_peak']:.1f}% of peak)")
        oe = bench_overlay_emb(tab, 100, hp, cpu_leg_s)
        result["overlay_emb"] = oe
        log_cpu_leg("overlay_emb", oe)
        log(f"OverlayEmb (a8): {oe['us_per_step']:.0f} us per build + backward of a 2,048-token sequence "
            f"({oe['slots_replaced']} slots replaced), {oe['device_us_per_step']:.1f} us of it on the device")
        ds = bench_damage_scan(tab, 20, hp, cpu_leg_s)
        result["damage_scan"] = ds
        log_cpu_leg("damage_scan", ds)
        log(f"damage scan: {ds['us_per_block_kernel']:.0f} us per 8M-token block on the device "
            f"({ds['lookups_per_s_kernel'] / 1e9:.1f} G lookups/s), {ds['s_per_block_end_to_end'] * 1e3:.1f} ms end "
            f"to end ({ds['s_per_block_end_to_end_int32_tokens'] * 1e3:.1f} ms from int32 tokens)")
        rf = bench_real_format(max(50, args.steps // 4), max(20, args.warmup // 4))
        result["forward_real_format"] = rf
        log(f"forward (real IQ4_NL format): {rf['us_per_launch']:.1f} us/launch, {rf['gb_per_s']:.0f} GB/s "
            f"algorithmic ({100 * rf['frac_of_hbm_peak']:.1f}% of peak)")
        pl = bench_ple(max(20, args.steps // 10), max(3, args.warmup // 20), cpu_leg_s)
        result["ple_forward"] = pl
        log_cpu_leg("ple_forward", pl)
        log(f"ple_forward: {pl['us_per_step']:.0f} us/step; its two GEMMs alone {pl['gemm_us']:.0f} us "
            f"({pl['gemm_tflops']:.1f} TFLOP/s fp32; hipBLASLt {pl['hipblaslt_gemm_us']:.0f} us), the rest "
            f"{pl['non_gemm_us']:.0f} us; forward + backward to emb {pl['us_forward_backward_to_emb']:.0f} us")
        x3 = pl["bf16x3"]
        log(f"ple_forward with bf16x3 GEMMs: {x3['us_per_step']:.0f} us/step; GEMMs {x3['gemm_us']:.0f} us "
            f"({x3['gemm_tflops']:.1f} TFLOP/s fp32-equivalent); forward + backward to emb "
            f"{x3['us_forward_backward_to_emb']:.0f} us")
        x6 = pl["bf16x6"]
        log(f"ple_forward with bf16x6 GEMMs: {x6['us_per_step']:.0f} us/step; GEMMs {x6['gemm_us']:.0f} us; "
            f"forward + backward to emb {x6['us_forward_backward_to_emb']:.0f} us; GEMM error / (|A||B|): fp32 "
            f"{pl['gemm_err_vs_fp64']:.2e}, hipBLASLt {pl['hipblaslt_gemm_err_vs_fp64']:.2e}, bf16x3 "
            f"{x3['gemm_err_vs_fp64']:.2e}, bf16x6 {x6['gemm_err_vs_fp64']:.2e}")

    if not args.no_cpu:
        calls[0]()  # outs[0] = the step on token batch 0 and residual set 0, which the CPU repeats
        torch.cuda.synchronize()
        cb = cpu_baseline(hp, tokens_np, res[0].cpu(), args.cpu_seconds)
        same = bool(torch.equal(cb.pop("result").view(torch.int16), outs[0].cpu().view(torch.int16)))
        cb["matches_gpu_output"] = same
        result["cpu_baseline_literal"] = cb.pop("literal")
        result["cpu_baseline_literal_config0"] = cb.pop("literal_config0")
        cb["gpu_speedup"] = result["value"] / cb["value"]
        result["cpu_baseline_literal"]["gpu_speedup"] = result["value"] / result["cpu_baseline_literal"]["value"]
        result["cpu_baseline"] = cb
        lit = result["cpu_baseline_literal"]
        log(f"cpu baseline, the reference's per-position loop: {lit['value']:.3g} rows/s on 1 thread; "
            f"identical output: {lit['matches_vectorized']}; on config 0: "
            f"{result['cpu_baseline_literal_config0']['value']:.3g} rows/s")
        log(f"cpu baseline: {cb['value']:.3g} rows/s on {cb['cores']} threads; identical output: {same}")
    else:
        result["cpu_baseline"] = None

    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
