"""bench.py's command-line contract, without a GPU: one GPU is what it
measures, so a larger --gpus exits with status 2 and a JSON line saying so;
the probe modes are listed in its help."""
from __future__ import annotations

import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    r = _bench("--gpus", "2")
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]


def test_help_lists_the_probe_modes():
    r = _bench("--help")
    assert r.returncode == 0
    for flag in ("--copy-probe", "--sampler", "--sampled-generate", "--prefill-only", "--no-graph", "--kv"):
        assert flag in r.stdout, flag
