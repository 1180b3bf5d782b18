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


def test_profiles_hold_the_traffic_the_bench_reports():
    """Every `roofline.traffic` the bench reads has its line in the committed
    PMC summaries, within a few percent above the launch's algorithmic bytes
    (a missing or stale summary fails here, not silently as null)."""
    sys.path.insert(0, str(ROOT))
    import bench

    def items(w, lm=None):
        its = bench.workload_items(w)
        return its if lm is None else [it for it in its if bool(it[5]) == lm]

    B = 16

    def batch_bytes(M, K):
        return bench.wbytes(M, K) + B * (2 * K + 4 * (K // 64)) + B * 4 * M

    cases = [
        ("sweep", "bfp8_sweep_kernel", bench.metric_bytes(items("sweep"))),  # the single launch
        ("lm_head", "bfp8_gemv_head_kernel", bench.kernel_bytes(items("lm_head", lm=True))),
        ("gemv", "rt_rows_gemv_kernel", bench.kernel_bytes(items("gemv"))),
        ("down", "rt_rows_gemv_kernel", bench.kernel_bytes(items("down"))),
        ("batch16", f"{bench.batch_kernel(3584, 1024)}@3584x1024", batch_bytes(3584, 1024)),
        ("batch16", f"{bench.batch_kernel(65536, 1024)}@65536x1024", batch_bytes(65536, 1024)),
    ]
    for workload, kernel, alg in cases:
        t = bench.read_traffic(workload, kernel)
        assert t is not None, (workload, kernel)
        # (up to 15 % above: the small B = 16 shape's workgroups each read their
        # copy of the split activations, counted once per XCD)
        assert 0.99 <= t / alg <= 1.15, (workload, kernel, t, alg, t / alg)
