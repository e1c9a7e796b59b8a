"""bench.py's command line on the CPU: it parses, and refuses more than one GPU."""

from __future__ import annotations

import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=120)


def test_help_parses():
    res = _run("--help")
    assert res.returncode == 0, res.stderr
    for flag in ("--config", "--format", "--backward", "--spin-up-s", "--no-library-compare"):
        assert flag in res.stdout


def test_more_than_one_gpu_is_refused_with_a_message():
    res = _run("--gpus", "2")
    assert res.returncode == 2, res.stderr
    line = json.loads(res.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]
