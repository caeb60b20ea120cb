"""bench.py's command-line contract that needs no GPU: a run asked for more than one GPU
exits non-zero with one JSON line that says why (the hot path has no cross-GPU part), and
--help lists the flags the driver passes."""
import json
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args],
                          capture_output=True, text=True, timeout=120, cwd=ROOT)


def test_more_than_one_gpu_is_refused():
    res = _bench("--gpus", "2", "--steps", "3", "--warmup", "1")
    assert res.returncode != 0
    line = json.loads(res.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]


def test_help_lists_the_driver_flags():
    res = _bench("--help")
    assert res.returncode == 0
    for flag in ("--gpus", "--steps", "--warmup"):
        assert flag in res.stdout
