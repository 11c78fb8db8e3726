"""The benchmark's contract pieces that need no GPU: one GPU only, and the
committed traffic profile it reads its ``roofline.traffic`` from."""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_bench_refuses_more_than_one_gpu():
    """``bench.py --gpus 2`` exits with status 2 and says why, before torch or
    the GPU is touched."""
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    assert "--gpus 2 is not supported" in r.stderr and "one" in r.stderr
    assert r.stdout == ""


def test_bench_reads_traffic_from_the_committed_profile():
    """The machine-readable lines of the committed rocprofv3 summary give the
    forward's and the damage scan's HBM bytes a launch: above the algorithmic
    bytes (whole 128-byte lines), within 2x of them."""
    sys.path.insert(0, str(ROOT))
    import bench

    fwd = bench.traffic_from_profile("forward_q8_cfg1")
    scan = bench.traffic_from_profile("damage_scan_bitmap")
    assert fwd is not None and scan is not None
    assert 170_000_384 < fwd < 2 * 170_000_384
    assert 170_000_000 < scan < 2 * 170_000_000
    assert bench.traffic_from_profile("no_such_kernel") is None
