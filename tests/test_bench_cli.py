"""bench.py's command-line contract that needs no GPU: this path runs on
one GPU, so --gpus above 1 exits with status 2 and says why, before torch
or the library is touched."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused_with_a_reason():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "ONE GPU" in r.stderr and "asked for 2" in r.stderr
    assert r.stdout.strip() == ""
