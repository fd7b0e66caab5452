"""bench.py's command line where it needs no GPU: a request for more than
one GPU is refused with a message and exit status 2 (this build measures a
single MI355X), before anything touches a device."""

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_refuses_several_gpus():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2", "--steps", "1"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2, (r.returncode, r.stderr[-500:])
    assert "one GPU" in r.stderr or "single MI355X" in r.stderr, r.stderr[-500:]
    assert r.stdout.strip() == "", "no bench line for a refused run"
