"""bench.py's command-line contract, checked without a GPU: it runs on one GPU
only (a larger --gpus exits with status 2 and says so), and every workload the
measurements use is selectable."""
import os
import subprocess
import sys

from conftest import ROOT

BENCH = os.path.join(ROOT, "bench.py")


def run(*args):
    return subprocess.run([sys.executable, BENCH, *args], capture_output=True, text=True, timeout=120)


def test_more_than_one_gpu_exits_with_a_message():
    r = run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""  # no JSON line for a run that was not made


def test_every_workload_is_selectable():
    r = run("--help")
    assert r.returncode == 0
    for w in ("c2", "c3", "c4", "c5", "c5b16", "stream", "staging", "dropin"):
        assert w in r.stdout, w
