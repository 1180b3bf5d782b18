"""bench.py's contract on the CPU: one GPU only, and the CPU baseline leg
(the reference's host bfp8_gemv from oracle/_ref, or the oracle's
restatement of it) timed with the OpenMP default and with one thread."""
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_cpu_baseline_reports_both_thread_counts():
    sys.path.insert(0, str(ROOT))
    import bench

    items = bench.workload_items("gemv")
    out = bench.cpu_baseline(items, seconds=0.2, single_seconds=0.2)
    if out is None:
        pytest.skip("no CPU baseline library built (make -C oracle)")
    assert out["unit"] == "GB/s" and out["value"] > 0 and out["cores"] >= 1
    assert out["kind"] in ("reference", "port")
    if out["kind"] == "reference":
        one = out["single_thread"]
        assert one["cores"] == 1 and one["value"] > 0
