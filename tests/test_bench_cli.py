"""bench.py's command line on the CPU: it measures one GPU and refuses more."""
import os
import subprocess
import sys

from conftest import ROOT


def test_bench_refuses_several_gpus():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "measures one GPU" in r.stderr
    assert r.stdout == ""  # no JSON line
