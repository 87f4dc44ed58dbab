"""bench.py's command line on the CPU: the multi-GPU refusal and the help text. Neither
path touches a GPU."""
import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run(*args):
    return subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), *args],
                          capture_output=True, text=True, timeout=120)


def test_more_than_one_gpu_is_refused():
    r = run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU only" in r.stderr
    assert r.stdout == ""  # no JSON line: no result is claimed


def test_help_lists_the_modes():
    r = run("--help")
    assert r.returncode == 0
    for flag in ("--config", "--suite", "--sweep", "--layers", "--profile-run",
                 "--traffic-summary", "--calibrate-copy"):
        assert flag in r.stdout, flag
