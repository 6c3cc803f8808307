"""bench.py's command-line contract on the CPU: more than one GPU is refused
with one JSON line that says so (the path is data-parallel across requests
and has no multi-GPU leg), before any device work."""

import json
import subprocess
import sys

from helpers import ROOT


def test_more_than_one_gpu_is_refused_with_a_message():
    for n in (2, 8):
        p = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", str(n)], capture_output=True, text=True,
                           timeout=300, cwd=ROOT)
        assert p.returncode == 2, p.stderr[-2000:]
        line = json.loads(p.stdout.strip().splitlines()[-1])
        assert line["n_gpus"] == n and "one GPU" in line["error"]
