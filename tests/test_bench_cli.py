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
                 "--traffic-summary", "--calibrate-copy", "--write-path"):
        assert flag in r.stdout, flag


def test_write_path_bytes():
    """The write path's byte model, counted by hand for two tokens of one sequence and one
    kv head at head_dim 4 with a 16-token K group: 2 x 2 x 4 x 2 B of fp16 rows read; INT4
    writes 2 x 2 x 2 B of codes, 2 x 4 B of V pairs and 4 x 4 B of K pairs (one group)."""
    sys.path.insert(0, REPO)
    import bench
    assert bench.write_path_bytes([2], "fp16", 16, hkv=1, d=4) == 64
    assert bench.write_path_bytes([2], "int4", 16, hkv=1, d=4) == 32 + 8 + 8 + 16
    assert bench.write_path_bytes([2], "int8", 16, hkv=1, d=4) == 32 + 16 + 8 + 16
    # a second sequence of 17 tokens opens two K groups
    assert bench.write_path_bytes([2, 17], "fp8", 16, hkv=1, d=4) == \
        19 * 16 + 19 * 8 + 19 * 4 + 3 * 16
