"""
bench.py's host side (no GPU): the HBM traffic each bench line reports comes from the committed
counter summaries under profiles/ (one figure per launch for the headline kernel, one per layer
for each batched workload, found by its workload name), and a run on more than one GPU is refused
with a message.
"""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_headline_traffic_is_near_its_algorithmic_bytes():
    t = bench.measured_traffic()
    # 8 int4 records of 3,342,336 B + the 256 KB router + x and out
    alg = 8 * 3_342_336 + 64 * 2048 * 2 + 2 * 2048 * 2
    assert t is not None and 1.0 <= t / alg <= 1.2, t


@pytest.mark.parametrize("name", sorted(bench.BATCH_SPECS))
def test_every_batched_workload_has_its_own_traffic(name):
    t = bench.measured_traffic(bench.BATCH_PROFILE, name)
    assert t is not None, name
    # the two GEMV kernels' bytes: at least most of a layer's distinct records (the smallest,
    # OLMoE mixed bs=8, runs ~140 MB of records per layer), and never another workload's figure
    others = {bench.measured_traffic(bench.BATCH_PROFILE, n) for n in bench.BATCH_SPECS if n != name}
    assert t > 100e6 and t not in others


def test_prefill_traffic_and_unknown_workload():
    assert bench.measured_traffic(bench.PREFILL_PROFILE) > 325_582_848  # above its algorithmic bytes
    assert bench.measured_traffic(bench.BATCH_PROFILE, "no-such-workload") is None
    assert bench.measured_traffic(ROOT / "profiles" / "no-such-file.md") is None


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=300, cwd=ROOT)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr) or "1 GPU" in (r.stdout + r.stderr), r.stdout + r.stderr
