"""bench.py's command-line contract that needs no GPU: it measures one GPU
and refuses a multi-GPU request with a message instead of a figure."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    assert "ONE GPU" in r.stderr + r.stdout
    assert r.stdout.strip() == ""  # no JSON line
