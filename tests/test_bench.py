"""bench.py's contract, checked on the CPU: the one-GPU exit, the per-row
algorithmic bytes behind ``achieved_gbs`` and ``roofline``, the layer
schedule it times, and the committed traffic record it reads.
"""

from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import bench  # noqa: E402  (stdlib-only at import time)
from oracle import sbda_oracle as ref  # noqa: E402


def test_multi_gpu_request_exits_with_a_message():
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                         capture_output=True, text=True, timeout=300, cwd=ROOT)
    assert res.returncode == 2
    assert "one GPU" in res.stderr
    assert res.stdout == ""


def test_algorithmic_bytes_are_the_metric_figures():
    # Per row: forward reads q, k, v and writes o (4 rows of D elements) plus
    # one fp32 log-normaliser; backward reads q, k, v, dO and writes dq, dk,
    # dv (7 rows) plus the log-normaliser read.
    assert bench.algorithmic_bytes(1, 64, 2) == (516, 900)
    assert bench.algorithmic_bytes(1, 64, 4) == (1028, 1796)   # the fp32 CPU baseline
    rows = 8 << 20                                              # B=1, H=8, T=2^20
    fwd, bwd = bench.algorithmic_bytes(rows, 64, 2)
    total = 20 * (fwd + bwd)
    assert total == 237_565_378_560
    assert total / 8e12 * 1e3 == pytest.approx(29.70, abs=0.01)   # ms at 8 TB/s
    # 226,560 bytes per position over the 20 layers: 35.31 M positions/s at 8 TB/s.
    assert bench.roofline_positions_per_s(8, 64, 20) == pytest.approx(8e12 / 226_560)
    assert bench.roofline_positions_per_s(8, 64, 20) / 1e6 == pytest.approx(35.31, abs=0.01)


def test_timed_schedule_is_the_sbda_route(sbda):
    for layer in range(1, 21):
        offs = bench.sbda_offsets(layer)
        assert offs == ref.sbda_layer_offsets(layer)
        assert offs == sbda.topology_offsets(layer, topology="sbda")
        assert len(offs) == (2 if layer <= 2 else 4)


def test_traffic_record_matches_the_workload():
    rec = json.loads(bench.TRAFFIC_FILE.read_text())
    assert (rec["length"], rec["heads"], rec["head_dim"], rec["dtype"]) == (1 << 20, 8, 64, "bf16")
    assert (ROOT / rec["source"]).exists()
    fwd_alg, bwd_alg = bench.algorithmic_bytes(rec["length"] * rec["heads"], rec["head_dim"], 2)
    for kind, alg in (("forward", fwd_alg), ("backward", bwd_alg)):
        assert rec[f"{kind}_algorithmic_bytes_per_launch"] == alg
        measured = rec[f"{kind}_bytes_per_launch"]
        assert measured == pytest.approx(rec[f"{kind}_read_bytes_per_launch"]
                                         + rec[f"{kind}_write_bytes_per_launch"])
        # Counter traffic bounds HBM bytes from above; it cannot undercut the
        # bytes the kernel must move, and re-reads beyond 1.5x would mean the
        # record is stale.
        assert 1.0 <= measured / alg < 1.5
