"""bench.py's command line on the CPU: one GPU only (`--gpus N` above 1 ends
with an explanation and a non-zero status before anything touches a GPU)."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2", "--steps", "1", "--warmup", "0"],
                       capture_output=True, text=True, cwd=ROOT, timeout=300)
    assert r.returncode == 2
    msg = r.stdout + r.stderr
    assert "one GPU" in msg and "--gpus 2" in msg
    assert not any(line.startswith("{") for line in r.stdout.splitlines())   # no bench line
