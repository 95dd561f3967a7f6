"""CPU checks of bench.py's contract and accounting (no GPU needed).

The roofline figures bench.py reports rest on two per-launch formulas: the
algorithmic FLOP of a prefill launch (2 * T * hidden * N) and the algorithmic
HBM bytes of a decode launch (weights + x + q/k/v + cos/sin rows + gammas +
positions, each once).  They are checked here against the figures worked out
independently from the BASELINE configurations: 1.0308e11 FLOP for the
Qwen3-8B B=4 x S=512 prefill, 1.718e11 for the 30B-A3B S=8192 prefill, and
51.68 MB for the Qwen3-8B B=64 decode step.
"""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_prefill_flop_per_launch():
    assert bench.flops(2048, 4096, 6144) == 2 * 2048 * 4096 * 6144
    assert abs(bench.flops(2048, 4096, 6144) - 1.0308e11) / 1.0308e11 < 1e-4
    assert abs(bench.flops(8192, 2048, 5120) - 1.718e11) / 1.718e11 < 1e-3


def test_decode_bytes_per_launch():
    b = bench.decode_bytes(64, 4096, 6144)
    weights = 6144 * 4096 * 2
    assert weights == 50331648                     # the 50.33 MB weight stream dominates
    assert abs(b - 51.68e6) / 51.68e6 < 2e-3
    # the terms beyond the weights: x (0.52 MB), outputs (0.79 MB), cos/sin rows, gammas, positions
    assert b - weights == 64 * 4096 * 2 + 64 * 6144 * 2 + 64 * 128 * 4 + 128 * 4 + 64 * 4


def test_more_than_one_gpu_is_refused():
    res = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True,
                         text=True, timeout=120)
    assert res.returncode == 2
    assert "one GPU" in res.stderr
    assert res.stdout.strip() == ""  # no JSON line for an unsupported run


def test_cpu_legs_report_well_formed_records():
    rec = bench.cpu_baseline(budget_s=0.0)
    assert set(rec) >= {"value", "unit", "cores", "kind", "sample"}
    assert rec["unit"] == "tokens/s" and rec["kind"] == "port" and rec["value"] > 0 and rec["cores"] >= 1
    tps, ms = bench.cpu_config1(reps=2)
    assert tps > 0 and ms > 0 and abs(tps - 128 / (ms * 1e-3)) / tps < 1e-6
