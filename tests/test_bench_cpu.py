"""CPU checks of bench.py's contract that need no GPU: the multi-GPU refusal
and the committed traffic summary the roofline reads."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr and r.stdout == ""


def test_traffic_summary_parses():
    sys.path.insert(0, ROOT)
    import bench
    t = bench.read_traffic()
    assert t is not None and 1e13 < t < 1e14  # the layer step's soft launches move ~24 TB
