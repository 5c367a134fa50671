"""bench.py's command-line contract that needs no GPU: more than one GPU is
refused with a message (this build measures one GPU), before torch or the
HIP library is touched."""
from __future__ import annotations

import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*args, env=None):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=120, env=env)


def test_more_than_one_gpu_is_refused():
    r = _bench("--gpus", "2", "--steps", "1")
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_world_size_above_one_is_refused():
    env = dict(os.environ, WORLD_SIZE="4")
    r = _bench("--steps", "1", env=env)
    assert r.returncode == 2
    assert "--gpus 1" in r.stderr
