"""bench.py's host-side parts, on the CPU: the one-GPU refusal, the traffic
figure read from the committed rocprofv3 summary, and the CPU baseline leg
(the oracle's C restatement timed on this host) with the fields its JSON
object carries."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, cwd=ROOT, timeout=300)
    assert r.returncode == 2
    assert "measures one GPU" in r.stderr
    assert r.stdout == ""


def test_traffic_figure_and_algorithmic_bytes():
    assert bench.algorithmic_bytes(bench.CFG2) == 2 * 1024 ** 3
    traffic = bench.read_traffic()
    assert isinstance(traffic, int)
    # HBM bytes per fused launch: the algorithmic bytes plus the block ids
    assert 0 <= traffic / bench.algorithmic_bytes(bench.CFG2) - 1 < 0.001


def test_cpu_baseline_leg():
    from oracle import native
    if not native.available():
        from oracle import build as obuild
        obuild.build()
    cpu = bench.run_cpu_baseline(bench.CFG2, budget_s=0.5)
    assert cpu["kind"] == "port" and cpu["unit"] == "reused KV tokens/s"
    assert cpu["value"] > 0 and cpu["GBps"] > 0
    assert 1 <= cpu["cores"] <= 16 and cpu["cores"] <= cpu["cores_available"]
    assert cpu["cpu_model"] and cpu["torch_version"]
    c1 = cpu["config1"]
    assert c1["value"] > 0 and c1["runs"] >= 5
    assert "OpenMP" in cpu["sample"] or "numpy" in cpu["sample"]
