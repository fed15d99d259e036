"""bench.py's command line on a CPU-only host: more than one GPU is refused
with a message (the verify step is measured on one GPU), and the help lists
the measurement modes."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args],
                          capture_output=True, text=True, timeout=120)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = _run("--gpus", "2")
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_help_lists_the_modes():
    r = _run("--help")
    assert r.returncode == 0
    for opt in ("--steps", "--warmup", "--workload", "--pmc-probe", "--pmc-probe-accept",
                "--pmc-probe-large", "--tune-gemms"):
        assert opt in r.stdout
