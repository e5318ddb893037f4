"""CPU checks of bench.py's command line contract (no GPU work)."""
import os
import subprocess
import sys

from conftest import ROOT


def test_multi_gpu_request_exits_with_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr
