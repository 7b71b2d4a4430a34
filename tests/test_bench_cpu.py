"""bench.py contract checks that need no GPU: every measurement leg exists, and N > 1 GPUs
exits with a message."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_measurement_legs_exist():
    sys.path.insert(0, ROOT)
    import bench
    for name in ("gemv_microbench", "copy_calibration", "cpu_baseline", "bench_batch4", "bench_long",
                 "bench_tokenizer", "step_timeline", "timeline_child", "main"):
        assert callable(getattr(bench, name)), name


def test_more_than_one_gpu_is_refused():
    out = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                         text=True, timeout=60)
    assert out.returncode == 2
    assert "one MI355X" in json.loads(out.stdout.strip().splitlines()[-1])["error"]
