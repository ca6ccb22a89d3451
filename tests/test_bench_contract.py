"""bench.py's command-line contract, on the CPU: one GPU only (more is refused
with a message and exit status 2 before anything touches a GPU), and the
documented options parse."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def run(*args):
    return subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                          timeout=120)


def test_more_than_one_gpu_is_refused_with_a_message():
    r = run("--gpus", "8", "--steps", "5", "--warmup", "1")
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_help_lists_the_legs():
    r = run("--help")
    assert r.returncode == 0
    for leg in ("head", "prefill", "qwen", "qlinear"):
        assert leg in r.stdout
